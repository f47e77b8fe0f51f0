"""GPU parity of the gfx950 B1_0 linear against the CPU oracle.

Bars (stated here, used below):
  EXACT mode  : bit-identical to the oracle's scalar path (the reference's
                src/b1_0_kernel.h:240-287 summation order).
  FAST modes  : per element |y - ref| / max(|ref|, rms(ref)) <= 1e-2 and
                cosine(y, ref) >= 0.9999, ref = fp64 brute force or the
                oracle's AVX2 path.
Full-size shapes use size-independent properties (exact scaling by 2,
exact negation under complemented sign words, sampled rows vs fp64).
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


def rel_to_rms(y, ref):
    ref = np.asarray(ref, dtype=np.float64)
    den = np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref)))
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref) / den))


def cosine(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b)))


def assert_fast_close(y, ref, what=""):
    r, c = rel_to_rms(y, ref), cosine(y, ref)
    say(f"  {what}: rel_to_rms={r:.3e} cos={c:.8f}")
    assert r <= TOL_REL, what
    assert c >= TOL_COS, what


def gpu_run(torch, b1, act, raw, n, mode, lda=None, ldo=None, nonfinite=None):
    m, k = act.shape
    if lda is None:
        a = torch.from_numpy(np.ascontiguousarray(act)).cuda()
    else:
        big = torch.zeros((m, lda), dtype=torch.float32)
        big[:, :k] = torch.from_numpy(act)
        a = big.cuda()[:, :k]
    w = torch.from_numpy(np.ascontiguousarray(raw).ravel()).cuda()
    out = None
    if ldo is not None:
        out = torch.full((m, ldo), 7.0, dtype=torch.float32, device="cuda")
    y = b1.linear(a, w, n, out=out, mode=mode, nonfinite=nonfinite)
    torch.cuda.synchronize()
    return y.cpu().numpy()


# ------------------------------------------------------ golden fixtures ----

def test_golden_exact_bit_exact(torch, b1):
    from tests.golden import make_golden
    for name, c in make_golden.load_all().items():
        say(f"golden exact {name}")
        y = gpu_run(torch, b1, c["act"], c["w"], int(c["n"]), "exact")
        assert np.array_equal(y.view(np.uint32), c["y_scalar"].view(np.uint32)), name


@pytest.mark.parametrize("mode", ["auto", "gemm", "gemv"])
def test_golden_fast(torch, b1, mode):
    from tests.golden import make_golden
    for name, c in make_golden.load_all().items():
        m, k = c["act"].shape
        if mode == "gemv" and (m > 16 or k % 64):
            continue
        if mode == "gemm" and k % 64:
            continue
        say(f"golden {mode} {name}")
        y = gpu_run(torch, b1, c["act"], c["w"], int(c["n"]), mode)
        assert_fast_close(y, c["y_f64"], f"{mode} {name}")


# ------------------------------------------------------------ configs ----

def test_c1_parity_config(torch, b1, oracle):
    """M=256, K=3072, N=3072: EXACT bit-exact vs the scalar oracle; FAST vs
    the AVX2 oracle (the reference's optimised path)."""
    from bonsai_b1 import synth
    m, k, n = 256, 3072, 3072
    act = synth.activations(m, k, 42)
    raw = synth.packed_weights(n, k, 43)
    say("c1 oracle scalar")
    ys, _ = oracle.linear(act, raw, n, variant="scalar", nth=16, nthreads=16)
    say("c1 gpu exact")
    ye = gpu_run(torch, b1, act, raw, n, "exact")
    assert np.array_equal(ye.view(np.uint32), ys.view(np.uint32))
    say("c1 oracle avx2")
    ya, _ = oracle.linear(act, raw, n, variant="avx2", nth=16, nthreads=16)
    for mode in ("auto", "gemm"):
        say(f"c1 gpu {mode}")
        assert_fast_close(gpu_run(torch, b1, act, raw, n, mode), ya, f"c1 {mode}")


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
def test_small_m_config(torch, b1, oracle, m):
    """Small-M GEMV shape: K=3072, N=18432."""
    from bonsai_b1 import synth
    k, n = 3072, 18432
    act = synth.activations(m, k, 100 + m)
    raw = synth.packed_weights(n, k, 200)
    ya, _ = oracle.linear(act, raw, n, variant="avx2", nth=16, nthreads=16)
    for mode in ("gemv", "gemm", "auto"):
        say(f"small-m M={m} {mode}")
        assert_fast_close(gpu_run(torch, b1, act, raw, n, mode), ya, f"M={m} {mode}")


@pytest.mark.parametrize("shape", [
    (4096, 3072, 12288),   # headline GEMM
    (4608, 3072, 9216),    # C3 fused QKV projection
    (4608, 3072, 3072),    # C3 out-projection
    (4608, 3072, 12288),   # C4 MLP up-projection
    (4608, 12288, 3072),   # C4 MLP down-projection
    (4608, 3072, 21504),   # C5 single-stream linear1
    (4608, 15360, 3072),   # C5 single-stream linear2
])
def test_full_size_properties(torch, b1, shape):
    from bonsai_b1 import synth
    m, k, n = shape
    say(f"full-size {shape}")
    a = synth.device_activations(m, k, 7)
    w = synth.device_packed_weights(n, k, 8)
    # keep activations out of the fp16 subnormal range, where fp16(2a) and
    # 2 fp16(a) round at different granularity
    a = torch.where(a.abs() < 2.0 ** -12, torch.zeros_like(a), a)
    y = b1.linear(a, w, n, mode="auto")
    # exact scaling of the activations: fp16(2a) = 2 fp16(a) for normal
    # fp16 values and the fp32 MFMA sums scale exactly
    y2 = b1.linear(a * 2.0, w, n, mode="auto")
    assert torch.equal(y2, 2.0 * y)
    # exact scaling of every fp16 block scale by 2 (exponent + 1)
    w2 = w.view(n, k // 32, 6).clone()
    sc = w2[:, :, 0:2].contiguous().view(torch.float16) * 2
    w2[:, :, 0:2] = sc.view(torch.uint8).view(n, k // 32, 2)
    y3 = b1.linear(a, w2.view(-1), n, mode="auto")
    assert torch.equal(y3, 2.0 * y)
    # complemented sign words: every expanded weight flips sign exactly; the
    # MFMA's internal rounding is not sign-symmetric bit for bit (measured:
    # a few ulp of the output), so the negation is checked to 1e-5 of
    # rms(y) -- one wrong sign (|scale * a| ~ 1e-2 rms) is 1000x larger
    wc = w.view(n, k // 32, 6).clone()
    wc[:, :, 2:6] ^= 0xFF
    yc = b1.linear(a, wc.view(-1), n, mode="auto")
    rms = float(y.pow(2).mean().sqrt())
    assert float((yc + y).abs().max()) <= 1e-5 * rms
    # sampled rows vs fp64
    rows = torch.linspace(0, m - 1, 24).long()
    from oracle import b1_oracle as o
    raw = w.cpu().numpy().reshape(n, -1)
    ref = o.linear_f64(a[rows].cpu().numpy(), raw, n)
    torch.cuda.synchronize()
    assert_fast_close(y[rows].cpu().numpy(), ref, f"{shape} sampled rows")


def test_exact_mode_full_size_agrees(torch, b1):
    from bonsai_b1 import synth
    m, k, n = 1024, 3072, 3072
    a = synth.device_activations(m, k, 17)
    w = synth.device_packed_weights(n, k, 18)
    ye = b1.linear(a, w, n, mode="exact")
    yf = b1.linear(a, w, n, mode="gemm")
    torch.cuda.synchronize()
    assert_fast_close(yf.cpu().numpy(), ye.cpu().numpy(), "gemm vs exact 1024x3072x3072")


# --------------------------------------------------------------- edges ----

def test_edges(torch, b1, oracle):
    from bonsai_b1 import capi, synth
    k, n = 256, 40
    act = synth.activations(5, k, 1)
    raw = synth.packed_weights(n, k, 2)
    ys, _ = oracle.linear(act, raw, n, variant="scalar")
    yf = oracle.linear_f64(act, raw, n)

    say("edge: M=0 is a no-op")
    a = torch.zeros((0, k), device="cuda")
    out = b1.linear(a, torch.from_numpy(raw.ravel()).cuda(), n)
    assert out.shape == (0, n)

    say("edge: strided rows (lda > K, ldo > N)")
    for mode in ("exact", "auto", "gemm", "gemv"):
        y = gpu_run(torch, b1, act, raw, n, mode, lda=k + 36, ldo=n + 24)
        if mode == "exact":
            assert np.array_equal(y[:, :n], ys)
        else:
            assert_fast_close(y[:, :n], yf, f"strided {mode}")
        assert np.all(y[:, n:] == 7.0), "columns beyond out_dim must be untouched"

    say("edge: K=32 (one block) and K=96 take the exact path in auto")
    for kk in (32, 96):
        a1 = synth.activations(3, kk, 5)
        r1 = synth.packed_weights(16, kk, 6)
        s1, _ = oracle.linear(a1, r1, 16, variant="scalar")
        assert np.array_equal(gpu_run(torch, b1, a1, r1, 16, "auto"), s1)
        with pytest.raises(b1.B1Error):
            gpu_run(torch, b1, a1, r1, 16, "gemm")

    say("edge: unaligned activation pointer")
    base = torch.zeros((5 * k + 1,), device="cuda")
    base[1:] = torch.from_numpy(act.ravel()).cuda()
    a_un = base[1:].view(5, k)
    wdev = torch.from_numpy(raw.ravel()).cuda()
    y = b1.linear(a_un, wdev, n, mode="auto")
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), ys)
    with pytest.raises(b1.B1Error) as ei:
        b1.linear(a_un, wdev, n, mode="gemm")
    assert ei.value.status == capi.ERR_ARG


@pytest.mark.parametrize("mode", ["exact", "gemm", "gemv"])
def test_nonfinite_counter(torch, b1, mode):
    """Replaces the reference's abort (src/b1_0_kernel.h:194-198): NaN in one
    activation row poisons that row; an Inf fp16 scale poisons a column."""
    from bonsai_b1 import synth
    m, k, n = 4, 128, 48
    act = synth.activations(m, k, 3)
    raw = synth.packed_weights(n, k, 4)
    ctr = torch.zeros(1, dtype=torch.int32, device="cuda")
    gpu_run(torch, b1, act, raw, n, mode, nonfinite=ctr)
    assert int(ctr.item()) == 0
    act[2, 7] = np.nan
    gpu_run(torch, b1, act, raw, n, mode, nonfinite=ctr)
    assert int(ctr.item()) == n
    ctr.zero_()
    act[2, 7] = 0.5
    r3 = raw.reshape(n, k // 32, 6).copy()
    r3[5, 2, 0:2] = [0x00, 0x7C]     # +Inf scale for row 5, block 2
    gpu_run(torch, b1, act, r3.reshape(n, -1), n, mode, nonfinite=ctr)
    assert int(ctr.item()) == m


@pytest.mark.parametrize("m,n", [(256, 1024), (200, 600)])
def test_nonfinite_counter_wide_tiles(torch, b1, m, n):
    """The staged GEMM's counter on full 128 x 512 tiles (vector-store path)
    and on ragged ones: a NaN activation poisons one output row, an Inf fp16
    scale one output column."""
    from bonsai_b1 import synth
    k = 768
    act = synth.activations(m, k, 5)
    raw = synth.packed_weights(n, k, 6)
    ctr = torch.zeros(1, dtype=torch.int32, device="cuda")
    gpu_run(torch, b1, act, raw, n, "gemm", nonfinite=ctr)
    assert int(ctr.item()) == 0
    act[130, 9] = np.nan
    gpu_run(torch, b1, act, raw, n, "gemm", nonfinite=ctr)
    assert int(ctr.item()) == n
    ctr.zero_()
    act[130, 9] = 0.25
    r3 = raw.reshape(n, k // 32, 6).copy()
    r3[517, 3, 0:2] = [0x00, 0x7C]   # +Inf scale for output column 517, block 3
    gpu_run(torch, b1, act, r3.reshape(n, -1), n, "gemm", nonfinite=ctr)
    assert int(ctr.item()) == m


def test_residency_builder_and_callback(torch, b1, oracle):
    """bonsai_b1_weights_upload + bonsai_b1_linear (b1_linear builder, fills
    the userdata) + the ggml-style callback over stand-in tensors."""
    import ctypes
    from bonsai_b1 import capi, synth
    m, k, n = 6, 512, 96
    act = synth.activations(m, k, 9)
    raw = synth.packed_weights(n, k, 10)
    ys, _ = oracle.linear(act, raw, n, variant="scalar")
    W = b1.Weights(raw, k, n)
    torch.cuda.synchronize()
    a = torch.from_numpy(act).cuda()
    ud = capi.B1LinearUserData()
    y = W.linear(a, mode="exact", ud=ud)
    torch.cuda.synchronize()
    assert (ud.magic, ud.in_dim, ud.out_dim) == (0x31423142, k, n)
    assert np.array_equal(y.cpu().numpy(), ys)

    class T(ctypes.Structure):
        pass
    T._fields_ = [("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                  ("src", ctypes.POINTER(T) * 2), ("data", ctypes.c_void_p)]
    out = torch.empty((m, n), device="cuda")
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
    ud2 = capi.B1LinearUserData(0x31423142, k, n)
    lib = b1.load()
    for ith in range(1, 4):        # other ggml tasks return at once
        lib.bonsai_b1_linear_f32_f32(ctypes.byref(td), ith, 4, ctypes.byref(ud2))
    lib.bonsai_b1_linear_f32_f32(ctypes.byref(td), 0, 4, ctypes.byref(ud2))
    torch.cuda.synchronize()
    assert_fast_close(out.cpu().numpy(), oracle.linear_f64(act, raw, n), "callback")
    W.free()


def test_callback_deferred_checking(torch, b1):
    """bonsai_b1_callback_defer(1): the callback enqueues each op without a
    host synchronisation; bonsai_b1_callback_finish synchronises once,
    reports the non-finite outputs of every op since the last finish and
    resets.  Outputs equal the library's AUTO linear."""
    import ctypes
    from bonsai_b1 import capi, synth
    m, k, n = 6, 512, 96
    act = synth.activations(m, k, 19)
    raw = synth.packed_weights(n, k, 20)
    W = b1.Weights(raw, k, n)
    a = torch.from_numpy(act).cuda()
    bad = act.copy()
    bad[2, 5] = np.inf                       # every output of token 2 is infinite
    abad = torch.from_numpy(bad).cuda()
    ref = W.linear(a).cpu().numpy()
    ref_bad = W.linear(abad).cpu().numpy()

    class T(ctypes.Structure):
        pass
    T._fields_ = [("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                  ("src", ctypes.POINTER(T) * 2), ("data", ctypes.c_void_p)]
    keep = []

    def node(x, o):
        ta, tw, td = T(), T(), T()
        ta.ne[:] = [k, m, 1, 1]
        ta.nb[:] = [4, 4 * k, 4 * k * m, 4 * k * m]
        ta.data = x.data_ptr()
        tw.ne[:] = [W.c.nbytes, 1, 1, 1]
        tw.data = W.c.data
        td.ne[:] = [n, m, 1, 1]
        td.nb[:] = [4, 4 * n, 4 * n * m, 4 * n * m]
        td.src[0] = ctypes.pointer(ta)
        td.src[1] = ctypes.pointer(tw)
        td.data = o.data_ptr()
        keep.extend([ta, tw, td])
        return td

    ud = capi.B1LinearUserData(0x31423142, k, n)
    lib = b1.load()
    torch.cuda.synchronize()
    cnt = ctypes.c_int32(-1)
    say("deferred callback: nothing pending")
    assert lib.bonsai_b1_callback_finish(ctypes.byref(cnt)) == capi.OK and cnt.value == 0
    assert lib.bonsai_b1_callback_defer(1) == capi.OK
    try:
        outs = [torch.full((m, n), 7.0, device="cuda") for _ in range(3)]
        say("deferred callback: three ops, the second with an infinite activation")
        for x, o in zip((a, abad, a), outs):
            lib.bonsai_b1_linear_f32_f32(ctypes.byref(node(x, o)), 0, 1, ctypes.byref(ud))
        assert lib.bonsai_b1_callback_finish(ctypes.byref(cnt)) == capi.ERR_NONFINITE
        assert cnt.value == n
        assert lib.bonsai_b1_callback_finish(ctypes.byref(cnt)) == capi.OK and cnt.value == 0
    finally:
        lib.bonsai_b1_callback_defer(0)
    y = [o.cpu().numpy() for o in outs]
    assert np.array_equal(y[0], ref) and np.array_equal(y[2], ref)
    assert np.array_equal(y[1].view(np.uint32), ref_bad.view(np.uint32))
    assert not np.isfinite(y[1][2]).any() and np.isfinite(np.delete(y[1], 2, axis=0)).all()
    say("per-op callback again")
    o = torch.empty((m, n), device="cuda")
    lib.bonsai_b1_linear_f32_f32(ctypes.byref(node(a, o)), 0, 1, ctypes.byref(ud))
    torch.cuda.synchronize()
    assert np.array_equal(o.cpu().numpy(), ref)
    W.free()


@pytest.mark.parametrize("m,n,ms,kind", [(4592, 12288, 4096, kd) for kd in
                                          ("plain", "scaled", "gate_residual", "swiglu", "gelu_packed")] +
                         [(4000, 9216, 3584, kd) for kd in ("plain", "gate_residual", "gelu_packed")])
def test_tail_rows_as_half_height_tiles(torch, b1, m, n, ms, kind):
    """M=4592 K=3072 N=12288 on 256 CUs runs its 768 full-round tiles of 128
    rows, then rows 4096..4591 as 64-row tiles in a second launch (M=4000
    N=9216: 504 tiles of rows [0, 3584) in two rounds, then the rest as
    64-row tiles).  Every output is the same sum in the same order as in two
    separate calls over rows [0, ms) and [ms, M), which take no such split:
    bit for bit, for each epilogue kind.  (The plain reference goes through the
    epilogue entry with no epilogue: the plain entry would split the
    ~500-row call along K.)  With range-safe row scales, the scaled rows
    equal the unscaled ones times their scales.  (M is a multiple of
    neither 128 nor 144, so no 16x16 tile kernel takes the plain forms.)"""
    from bonsai_b1 import synth
    k = 3072
    say(f"tail rows as half-height tiles: ({m},{k},{n}) {kind} "
        f"({torch.cuda.get_device_properties(0).multi_processor_count} CUs)")
    a = synth.device_activations(m, k, 61)
    w = synth.device_packed_weights(n, k, 62)
    if kind == "scaled":
        a[10] *= 3.0e5
        a[ms + 104] *= 2.0e6
        pa, rsc = b1.pack_act_f16_scaled(a)
    else:
        pa = b1.pack_act_f16(a)
    rb = k * 2                                   # packed bytes per row

    def run(rows, r0, whole=False):
        p = pa[r0 * rb:(r0 + rows) * rb]
        if kind == "plain":
            if whole:
                return b1.linear_packed_f16(p, w, k, n, rows)
            return b1.linear_packed_f16_epi(p, w, k, n, rows, "none")
        if kind == "gate_residual":
            return b1.linear_packed_f16_epi(p, w, k, n, rows, "gate_residual", gate=gate, residual=res[r0:r0 + rows])
        if kind == "swiglu":
            return b1.linear_packed_f16_epi(p, w, k, n, rows, "swiglu")
        _, po = b1.linear_packed_f16_to_packed(p, w, k, n, rows, 0, "gelu_tanh")
        return po

    g = torch.Generator(device="cuda").manual_seed(63)
    gate = 0.1 * torch.randn(n, device="cuda", generator=g)
    res = torch.randn((m, n), device="cuda", generator=g)
    if kind == "scaled":
        # the scaled entry splits a 512-row call along K too; its rows are the
        # unscaled products times their scales, one fp32 multiply each
        full = b1.linear_packed_f16_scaled(pa, rsc, w, k, n, m)
        ref = b1.linear_packed_f16_epi(pa, w, k, n, m, "none") * rsc[:, None]
        torch.cuda.synchronize()
        assert bool((rsc[ms:] != 1.0).any()), "a tail row needs a row scale"
        assert torch.equal(full.view(torch.uint8), ref.view(torch.uint8)), kind
        return
    full = run(m, 0, whole=True)
    head, tail = run(ms, 0), run(m - ms, ms)
    torch.cuda.synchronize()
    joined = torch.cat([head.reshape(-1), tail.reshape(-1)])
    assert torch.equal(full.reshape(-1).view(torch.uint8), joined.view(torch.uint8)), kind


@pytest.mark.parametrize("mode,m", [("gemv", 8), ("gemm", 256), ("gemm", 4608)])
def test_graph_replay_matches_eager(torch, b1, mode, m):
    """Launches captured into a HIP graph (as the benchmark does) with the
    caller's workspace give the eager result on every replay, with eager
    work between replays; m=4608 runs more than one round of persistent
    tiles per work-group."""
    from bonsai_b1 import synth
    k, n = 3072, 4096
    a = synth.device_activations(m, k, 31)
    w = synth.device_packed_weights(n, k, 32)
    ws = torch.empty(max(b1.workspace_bytes(m, k, n, mode), 16), dtype=torch.uint8, device="cuda")
    ref = b1.linear(a, w, n, mode=mode, workspace=ws).clone()
    y = torch.empty((m, n), device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        b1.linear(a, w, n, out=y, mode=mode, workspace=ws)
    for i in range(4):
        y.fill_(float(i + 1))
        b1.linear(a * 0.5, w, n, mode=mode, workspace=ws)   # unrelated eager work
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, ref), f"replay {i}"


# ------------------------------------------- packed-activation entry points --

def test_pack_act_layout_bit_exact(torch, b1, oracle):
    """bonsai_b1_pack_act_f16: word 16j+d of row m = fp16(a[m][32j+d]) |
    fp16(a[m][32j+d+16]) << 16, fp16 rounded to nearest even (the oracle's
    conversion, itself pinned exhaustively against F16C)."""
    rng = np.random.default_rng(5)
    m, k = 5, 384
    a = rng.standard_normal((m, k)).astype(np.float32)
    # rounding ties and near-ties, fp16 subnormals, signed zero, range edges
    h = (np.arange(1, 1 + k, dtype=np.uint16) * 7 + 0x3C00).view(np.float16)
    up = h.astype(np.float32).view(np.uint32) + (1 << 12)  # midpoints between fp16 neighbours
    a[1] = up.view(np.float32)
    a[2] = (up + 1).view(np.float32)                       # just above a tie
    a[3] = rng.uniform(-6e-5, 6e-5, k).astype(np.float32)  # subnormal range
    a[4, :8] = [0.0, -0.0, 65504.0, -65504.0, 65519.0, 6.1035156e-05, -5.96e-08, 2.98e-08]
    d = torch.from_numpy(a).cuda()
    packed = b1.pack_act_f16(d)
    torch.cuda.synchronize()
    got = packed.cpu().numpy().view(np.uint32).reshape(m, k // 2)
    hb = oracle.fp32_to_fp16_bits(a).reshape(m, k // 32, 32).astype(np.uint32)
    want = (hb[:, :, :16] | (hb[:, :, 16:] << 16)).reshape(m, k // 2)
    say(f"  pack: {int((got != want).sum())} mismatching words of {got.size}")
    assert np.array_equal(got, want)


def pack_area_bytes(m, k):
    """The range-safe packing of an fp32 call: m*k fp16 values, then m row
    scales, each area rounded up to 256 bytes."""
    return (m * k * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256


def unsplit_linear(torch, b1, a, w, n, mode):
    """The fp32 entry with a workspace that holds the packing only, so the
    GEMM runs unsplit along K."""
    ws = torch.empty(pack_area_bytes(*a.shape), dtype=torch.uint8, device="cuda")
    return b1.linear(a, w, n, mode=mode, workspace=ws)


@pytest.mark.parametrize("m,k,n", [(200, 768, 600), (128, 384, 512), (1, 384, 40)])
def test_linear_packed_matches_fused_entry(torch, b1, m, k, n):
    """pack + linear_packed gives bit-for-bit what bonsai_b1_linear_f32 gives
    in GEMM mode (same kernels, split along K the same way), including a
    padded output stride."""
    from bonsai_b1 import synth
    a = synth.device_activations(m, k, 41)
    w = synth.device_packed_weights(n, k, 42)
    ref = b1.linear(a, w, n, mode="gemm")
    out = torch.full((m, n + 12), 7.0, device="cuda")
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    packed = b1.pack_act_f16(a)
    b1.linear_packed_f16(packed, w, k, n, m, out=out[:, :n], nonfinite=nf)
    torch.cuda.synchronize()
    say(f"  packed ({m},{k},{n}): max |diff| {float((out[:, :n] - ref).abs().max()):.3e}")
    assert torch.equal(out[:, :n], ref)
    assert bool((out[:, n:] == 7.0).all()), "columns past out_dim untouched"
    assert int(nf.item()) == 0


@pytest.mark.parametrize("m,k,n,mode", [(1, 3072, 18432, "gemv"), (8, 3072, 18432, "gemv"), (16, 3072, 1000, "gemv"),
                                         (5, 768, 48, "gemv"), (3, 1536, 4000, "gemv"), (8, 1152, 500, "gemm")])
def test_linear_packed_small_m(torch, b1, m, k, n, mode):
    """Packed activations with M <= 16 run the small-M kernel (fragments
    loaded straight from the packing) and give bit for bit what the fp32
    entry's small-M kernel gives; K % 256 != 0 stays on the GEMM tile and
    matches GEMM mode."""
    from bonsai_b1 import synth
    say(f"packed small-M ({m},{k},{n}) vs {mode}")
    a = synth.device_activations(m, k, 43)
    w = synth.device_packed_weights(n, k, 44)
    ref = b1.linear(a, w, n, mode=mode)
    out = torch.full((m, n + 12), 7.0, device="cuda")
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    packed = b1.pack_act_f16(a)
    b1.linear_packed_f16(packed, w, k, n, m, out=out[:, :n], nonfinite=nf)
    torch.cuda.synchronize()
    say(f"  max |diff| {float((out[:, :n] - ref).abs().max()):.3e}")
    assert torch.equal(out[:, :n], ref)
    assert bool((out[:, n:] == 7.0).all()), "columns past out_dim untouched"
    assert int(nf.item()) == 0


@pytest.mark.parametrize("m,k,n", [(8, 768, 96), (160, 768, 600)])
def test_signed_scales(torch, b1, oracle, m, k, n):
    """fp16 scales of either sign (and +-0): the reference multiplies the
    signed scale into +-a (src/b1_0_kernel.h:125-134,253-277), so a negative
    scale flips every weight of its block.  EXACT is bit-exact vs the
    scalar oracle, FAST modes within the stated tolerance of fp64."""
    from bonsai_b1 import synth
    rng = np.random.default_rng(11)
    act = rng.standard_normal((m, k)).astype(np.float32)
    raw = synth.packed_weights(n, k, 12).reshape(n, k // 32, 6).copy()
    sc = raw[:, :, 0:2].copy().view("<u2")[..., 0]
    sc |= (rng.integers(0, 2, sc.shape) << 15).astype(np.uint16)     # random sign
    sc[0, :4] = [0x0000, 0x8000, 0x0000, 0x8000]                      # signed zeros
    raw[:, :, 0:2] = sc.astype("<u2").view(np.uint8).reshape(n, k // 32, 2)
    raw = raw.reshape(n, -1)
    want_scalar, bad = oracle.linear(act, raw, n, variant="scalar")
    assert bad == 0
    y = gpu_run(torch, b1, act, raw, n, "exact")
    assert np.array_equal(y.view(np.uint32), want_scalar.view(np.uint32))
    ref = oracle.linear_f64(act, raw, n)
    for mode in (["auto", "gemv", "gemm"] if m <= 16 else ["auto", "gemm"]):
        y = gpu_run(torch, b1, act, raw, n, mode)
        assert_fast_close(y, ref, f"signed scales {mode} ({m},{k},{n})")


# ------------------------------------------------------------ B1_0 writer --

@pytest.mark.parametrize("order", ["numpy", "sequential"])
def test_quantize_matches_reference_writers(torch, b1, oracle, order):
    """bonsai_b1_quantize_f32 reproduces each reference writer bit for bit:
    numpy's np.mean order (convert_to_b1_0_packed.py) and the left-to-right
    order (tests/c_ops/test_b1_linear.cpp), including the rare blocks where
    the two disagree, signed zeros, ties and a padded row stride."""
    rng = np.random.default_rng(21)
    w = rng.standard_normal((1000, 3200)).astype(np.float32)          # orders differ on ~9 blocks
    w[0, :64] = 0.0
    w[1, :32] = -0.0
    w[2, :] = (rng.integers(-3, 4, 3200) * 0.0009765625).astype(np.float32)
    w[3, :32] = np.float32(1e-40)                                      # subnormal magnitudes
    big = torch.zeros((1000, 3200 + 32), dtype=torch.float32)
    big[:, :3200] = torch.from_numpy(w)
    dw = big.cuda()[:, :3200]
    got = b1.quantize_f32(dw, order=order)
    torch.cuda.synchronize()
    want = oracle.pack(w, order=order)
    nbad = int((got.cpu().numpy() != want).sum())
    say(f"  quantize {order}: {nbad} differing bytes")
    assert nbad == 0


# -------------------------------------------------------------- GELU-tanh --

GELU_TOL = 1e-6  # |y - gelu64(x)| <= GELU_TOL * max(1, |x|); the fp32 exp2/reciprocal form is within 3e-7


def gelu64(x):
    from oracle import b1_oracle
    return b1_oracle.gelu_tanh_f64(x)


def gelu_inputs(rows, cols, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, cols)) * 3).astype(np.float32)
    x[0, :12] = [0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0, 100.0, -100.0, 1e4, -1e4, 3e-8, -5.5]
    return x


def test_gelu_tanh_matches_float64(torch, b1):
    x = gelu_inputs(37, 1028, 3)
    big = torch.zeros((37, 1032), dtype=torch.float32)
    big[:, :1028] = torch.from_numpy(x)
    dx = big.cuda()[:, :1028]
    y = b1.gelu_tanh(dx)
    b1.gelu_tanh(dx, out=dx)                                     # in place
    torch.cuda.synchronize()
    ref = gelu64(x)
    for got in (y.cpu().numpy(), dx.cpu().numpy()):
        err = np.abs(got.astype(np.float64) - ref) / np.maximum(1.0, np.abs(x))
        say(f"  gelu max scaled err {err.max():.2e}")
        assert err.max() <= GELU_TOL
    assert bool((big[:, 1028:] == 0).all()), "padding untouched"


def test_gelu_tanh_c4_size_matches_float64(torch, b1):
    """The standalone GELU at the size the C4 MLP runs it (4608 x 12288, the
    up-projection's output): 64 sampled rows, every element, within
    GELU_TOL * max(1, |x|) of the float64 GELU; the rest of the matrix
    finite and odd-symmetric in the sense gelu(x) - gelu(-x) = x (checked
    on one more sampled block by a second launch over -x)."""
    m, n = 4608, 12288
    g = torch.Generator(device="cuda")
    g.manual_seed(77)
    x = torch.randn((m, n), device="cuda", generator=g) * 3
    y = b1.gelu_tanh(x)
    yn = b1.gelu_tanh(-x)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(y).all())
    rows = np.random.default_rng(78).choice(m, 64, replace=False)
    xs = x[rows].cpu().numpy()
    err = np.abs(y[rows].cpu().numpy().astype(np.float64) - gelu64(xs)) / np.maximum(1.0, np.abs(xs))
    say(f"  C4-size gelu, 64 sampled rows: max scaled err {err.max():.2e}")
    assert err.max() <= GELU_TOL
    # gelu(x) - gelu(-x) = x exactly in real arithmetic; in fp32 within the
    # two evaluations' error bounds
    d = (y - yn - x).abs() / torch.clamp(x.abs(), min=1.0)
    assert float(d.max()) <= 2 * GELU_TOL + 2 ** -23


def test_gelu_pack_matches_pack_of_gelu(torch, b1, oracle):
    """gelu_tanh_pack_f16 == the pack_act_f16 layout of fp16(gelu(x)): each
    fp16 is within half an fp16 ulp (its rounding) plus the fp32 GELU bound
    GELU_TOL * max(1, |x|) of the float64 GELU.  The second term dominates
    in the fp16 subnormal range (large negative x, tiny outputs)."""
    m, k = 6, 768
    x = gelu_inputs(m, k, 4)
    packed = b1.gelu_tanh_pack_f16(torch.from_numpy(x).cuda())
    torch.cuda.synchronize()
    got = packed.cpu().numpy().view(np.uint32).reshape(m, k // 32, 16)
    lo = (got & 0xFFFF).astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (got >> 16).astype(np.uint16).view(np.float16).astype(np.float64)
    vals = np.concatenate([lo, hi], axis=-1).reshape(m, k)     # back to element order
    ref = gelu64(x)
    ulp = np.spacing(np.abs(ref).astype(np.float16)).astype(np.float64)
    err = np.abs(vals - ref) - (0.5 * ulp + GELU_TOL * np.maximum(1.0, np.abs(x)))
    say(f"  gelu pack worst margin {err.max():.2e}")
    assert err.max() <= 0


# --------------------------------------------------------- batched dispatch --

@pytest.mark.parametrize("mode", ["auto", "exact"])
def test_linear_batch_matches_single_calls(torch, b1, mode):
    """bonsai_b1_linear_batch == the same linears issued one by one (bit for
    bit: same kernels), over q/k/v sharing one input, a small-M op, a K the
    packed GEMM does not take (K % 384 != 0), a K % 64 != 0 op, and an op
    that overwrites a packed input before the next op reads it."""
    from bonsai_b1 import synth
    def w(n, k, seed):
        return synth.device_packed_weights(n, k, seed)
    x = synth.device_activations(200, 768, 1)
    y = synth.device_activations(200, 768, 2)
    z = synth.device_activations(8, 3072, 3)
    u = synth.device_activations(64, 96, 4)
    v = synth.device_activations(130, 640, 5)
    spec = [(x, w(600, 768, 10), 600), (x, w(300, 768, 11), 300), (x, w(40, 768, 12), 40),
            (y, w(768, 768, 13), 768), (z, w(96, 3072, 14), 96), (u, w(32, 96, 15), 32),
            (v, w(100, 640, 16), 100)]
    x_over = x.clone()
    ops = []
    outs = [torch.full((a.shape[0], n + 4), 7.0, device="cuda")[:, :n] for a, _, n in spec]
    for (a, wt, n), o in zip(spec, outs):
        ops.append((a, b1.device_weights(wt, a.shape[1], n), o))
    # 7: packed read of x_over (the packing is now of x_over)
    x_before = torch.empty((200, 40), device="cuda")
    ops.append((x_over, b1.device_weights(spec[2][1], 768, 40), x_before))
    # 8: a small-M op (no packing) writes rows 0..7 of x_over
    w_over = w(768, 3072, 17)
    ops.append((z, b1.device_weights(w_over, 3072, 768), x_over[:8]))
    # 9: reads x_over again: the stale packing must not be reused
    o8 = torch.empty((200, 600), device="cuda")
    ops.append((x_over, b1.device_weights(spec[0][1], 768, 600), o8))
    # 10, 11: a grouped small-M run on z (8 tokens, read as fp32: no packing)
    # whose SECOND op writes rows 8..15 of x_over; 12 reads x_over again, so
    # the packing made for op 9 must be dropped for every op of the group
    w_side = w(256, 3072, 18)
    side = torch.empty((8, 256), device="cuda")
    ops.append((z, b1.device_weights(w_side, 3072, 256), side))
    w_over2 = w(768, 3072, 19)
    ops.append((z, b1.device_weights(w_over2, 3072, 768), x_over[8:16]))
    o12 = torch.empty((200, 600), device="cuda")
    ops.append((x_over, b1.device_weights(spec[0][1], 768, 600), o12))
    b1.linear_batch(ops, mode=mode)
    torch.cuda.synchronize()
    for i, ((a, wt, n), o) in enumerate(zip(spec, outs)):
        ref = b1.linear(a, wt, n, mode=mode)
        torch.cuda.synchronize()
        assert torch.equal(o, ref), f"op {i}"
    ref_before = b1.linear(x, spec[2][1], 40, mode=mode)
    new_x = x.clone()
    b1.linear(z, w_over, 768, out=new_x[:8], mode=mode)
    ref8 = b1.linear(new_x, spec[0][1], 600, mode=mode)
    ref_side = b1.linear(z, w_side, 256, mode=mode)
    b1.linear(z, w_over2, 768, out=new_x[8:16], mode=mode)
    ref12 = b1.linear(new_x, spec[0][1], 600, mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(x_before, ref_before)
    assert torch.equal(x_over, new_x)
    assert torch.equal(o8, ref8)
    assert torch.equal(side, ref_side)
    assert torch.equal(o12, ref12), "a grouped op's output left a stale packing in use"


def test_linear_batch_fuses_concatenated_qkv(torch, b1):
    """q/k/v with weights as adjacent row ranges of one buffer and outputs as
    adjacent column ranges of one tensor run as one GEMM over the
    concatenated rows (bit for bit the three linears, which compute every
    output column the same way); bonsai_b1_weights_concat builds that buffer
    from separate device weights.  An op whose output overwrites the shared
    input is not fused."""
    import ctypes
    from bonsai_b1 import capi, synth
    m, k, n = 512, 3072, 1024
    x = synth.device_activations(m, k, 91)
    parts = [synth.device_packed_weights(n, k, 92 + i) for i in range(3)]
    lib = b1.load()
    cs = (capi.B1WeightsC * 3)(*[b1.device_weights(p, k, n) for p in parts])
    cat = capi.B1WeightsC()
    assert lib.bonsai_b1_weights_concat(cs, 3, None, ctypes.byref(cat)) == capi.OK
    torch.cuda.synchronize()
    assert cat.out_dim == 3 * n and cat.nbytes == 3 * parts[0].numel()
    catd = torch.empty(cat.nbytes, dtype=torch.uint8, device="cuda")
    import glob
    import os
    hip = ctypes.CDLL(sorted(glob.glob(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so*")))[0])
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(catd.data_ptr(), cat.data, cat.nbytes, 3) == 0     # device to device
    assert torch.equal(catd, torch.cat([p.reshape(-1) for p in parts]))
    rs = (k // 32) * 6
    views = [capi.B1WeightsC(cat.data + i * n * rs, k, n, n * rs, cat.device) for i in range(3)]
    qkv = torch.full((m, 3 * n + 4), 7.0, device="cuda")
    ops = [(x, views[i], qkv[:, i * n:(i + 1) * n]) for i in range(3)]
    b1.linear_batch(ops)
    torch.cuda.synchronize()
    for i in range(3):
        ref = b1.linear(x, parts[i], n)
        torch.cuda.synchronize()
        assert torch.equal(qkv[:, i * n:(i + 1) * n], ref), i
    assert bool((qkv[:, 3 * n:] == 7.0).all())
    # the first output overwrites the input the others read: run in order
    xx = torch.empty((m, 3 * n), device="cuda")
    xx[:, :k] = x
    a_in = xx[:, :k]
    ops2 = [(a_in, views[0], xx[:, :n]), (a_in, views[1], xx[:, n:2 * n]), (a_in, views[2], xx[:, 2 * n:3 * n])]
    b1.linear_batch(ops2)
    x0 = x.clone()
    y0 = b1.linear(x0, parts[0], n)
    x1 = x0.clone()
    x1[:, :n] = y0
    y1 = b1.linear(x1, parts[1], n)
    x2 = x1.clone()
    x2[:, n:2 * n] = y1
    y2 = b1.linear(x2, parts[2], n)
    torch.cuda.synchronize()
    assert torch.equal(xx[:, :n], y0) and torch.equal(xx[:, n:2 * n], y1) and torch.equal(xx[:, 2 * n:], y2)
    assert lib.bonsai_b1_weights_free(ctypes.byref(cat)) == capi.OK


GROUP_CASES = [  # (m, k, output widths): consecutive small-M ops on one input
    (1, 3072, [18432, 18432, 9216, 6144]),            # a step's modulation projections
    (5, 1536, [1000, 48, 4096, 16, 777, 1024, 3000, 2048, 500]),  # 8 grouped + 1 alone
    (16, 256, [64, 96]),
    (1, 3072, [18432] * 8),                           # more row groups than one pass of the CUs holds
    (8, 3072, [18432, 18432, 9216, 6144]),            # 8 token slots: fewer row groups per work-group
]


@pytest.mark.parametrize("m,k,ns", GROUP_CASES)
def test_linear_batch_groups_small_m_ops(torch, b1, oracle, m, k, ns):
    """Consecutive small-M ops on the same input run as one launch (up to
    8), from the fp32 rows at M <= 8 (no workspace) and over one range-safe
    packing above (the workspace that packing): each output bit for bit the
    op's own small-M call, the counter of non-finite outputs unchanged;
    within the FAST bar of the float64 oracle."""
    from bonsai_b1 import capi, synth
    say(f"group m={m} k={k} ns={ns}")
    x = synth.device_activations(m, k, 300 + m)
    ws = [synth.device_packed_weights(n, k, 310 + i) for i, n in enumerate(ns)]
    outs = [torch.full((m, n + 8), 7.0, device="cuda")[:, :n] for n in ns]
    ops = [(x, b1.device_weights(w, k, n), o) for w, n, o in zip(ws, ns, outs)]
    pack = (m * k * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256
    assert capi.linear_batch_workspace_bytes(ops) == (pack if m > 8 else 0)
    assert capi.linear_batch_workspace_bytes(ops[:1]) == 0       # alone: converts itself
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    b1.linear_batch(ops, nonfinite=nf)
    torch.cuda.synchronize()
    assert int(nf.item()) == 0
    for i, (w, n, o) in enumerate(zip(ws, ns, outs)):
        ref = b1.linear(x, w, n)
        torch.cuda.synchronize()
        assert torch.equal(o, ref), f"op {i}"
        assert bool((o.as_strided((m, 8), (o.stride(0), 1), o.storage_offset() + n) == 7.0).all()), f"op {i} pad"
    xh = x.cpu().numpy()
    for i in (0, len(ns) - 1):
        raw = ws[i].cpu().numpy()
        assert_fast_close(outs[i].cpu().numpy(), oracle.linear_f64(xh, raw, ns[i]), f"group op {i} vs fp64")


@pytest.mark.parametrize("seed", range(10))
def test_linear_batch_groups_random(torch, b1, oracle, seed):
    """Seeded random groupings of small-M ops (1-8 ops, output widths 1 to
    5000 rows, M 1-16, K a multiple of 256 up to 3072): each op's output bit
    for bit its own small-M call, the padding after each output row
    untouched, the last op within the FAST bar of the float64 oracle.  Op
    widths that are not multiples of 16 put partial row groups at every op
    boundary, and the op count and widths vary the work-groups per op."""
    from bonsai_b1 import synth
    rng = np.random.default_rng(1000 + seed)
    m = int(rng.integers(1, 17))
    k = 256 * int(rng.integers(1, 13))
    nops = int(rng.integers(1, 9))
    ns = [int(rng.choice([rng.integers(1, 64), rng.integers(64, 5001)])) for _ in range(nops)]
    say(f"random group seed={seed} m={m} k={k} ns={ns}")
    x = synth.device_activations(m, k, 700 + seed)
    ws = [synth.device_packed_weights(n, k, 710 + 10 * seed + i) for i, n in enumerate(ns)]
    outs = [torch.full((m, n + 3), 5.0, device="cuda")[:, :n] for n in ns]
    b1.linear_batch([(x, b1.device_weights(w, k, n), o) for w, n, o in zip(ws, ns, outs)])
    torch.cuda.synchronize()
    for i, (w, n, o) in enumerate(zip(ws, ns, outs)):
        ref = b1.linear(x, w, n)
        torch.cuda.synchronize()
        assert torch.equal(o, ref), f"op {i} (n={n})"
        pad = o.as_strided((m, 3), (o.stride(0), 1), o.storage_offset() + n)
        assert bool((pad == 5.0).all()), f"op {i} pad"
    assert_fast_close(outs[-1].cpu().numpy(), oracle.linear_f64(x.cpu().numpy(), ws[-1].cpu().numpy(), ns[-1]),
                      f"random group last op vs fp64 (seed {seed})")


@pytest.mark.parametrize("m", [1, 2, 4, 5, 8])
def test_linear_batch_group_fp32_rows(torch, b1, m):
    """A grouped run of at most 8 tokens reads the fp32 rows itself: with
    rows beyond the fp16 range (x 1e5, and 3e38 whose outputs overflow fp32)
    each op's outputs equal its own fp32 call bit for bit (those rows again
    in EXACT arithmetic) and the non-finite outputs are counted once; a row
    stride other than K (16-byte aligned) takes the same path, an unaligned
    view runs each op alone, both with no workspace."""
    from bonsai_b1 import capi, synth
    k, ns = 3072, [1024, 77, 2048]
    say(f"fp32 group m={m} k={k} ns={ns}")
    x = synth.device_activations(m, k, 450 + m)
    ws = [synth.device_packed_weights(n, k, 460 + i) for i, n in enumerate(ns)]
    dws = [b1.device_weights(w, k, n) for w, n in zip(ws, ns)]

    def run(xv):
        outs = [torch.full((m, n), 3.0, device="cuda") for n in ns]
        nf = torch.zeros(1, dtype=torch.int32, device="cuda")
        b1.linear_batch([(xv, dw, o) for dw, o in zip(dws, outs)], nonfinite=nf)
        refs = [b1.linear(xv, w, n) for w, n in zip(ws, ns)]
        torch.cuda.synchronize()
        for i, (o, r) in enumerate(zip(outs, refs)):   # equal, NaN where the call gives NaN
            assert torch.allclose(o, r, rtol=0.0, atol=0.0, equal_nan=True), f"op {i}"
        return outs, int(nf.item())

    xb = x.clone()
    xb[0] *= 1e5
    _, nf = run(xb)
    assert nf == 0
    if m >= 2:
        xb[m - 1] = 3.0e38
        outs, nf = run(xb)
        bad = sum(int((~torch.isfinite(o)).sum()) for o in outs)
        say(f"  non-finite outputs {bad}, counted {nf}")
        assert bad > 0 and nf == bad and all(bool(torch.isfinite(o[:m - 1]).all()) for o in outs)
    big = torch.zeros((m, k + 12), device="cuda")
    for off in (4, 1):
        xv = big[:, off:off + k]
        xv.copy_(x)
        ops = [(xv, dw, torch.empty((m, n), device="cuda")) for dw, n in zip(dws, ns)]
        assert capi.linear_batch_workspace_bytes(ops) == 0, f"offset {off}"
        run(xv)


def test_linear_batch_group_order_and_range(torch, b1):
    """Small-M ops whose outputs overlap one another or the shared input are
    not grouped (the batch keeps their order); a row beyond the fp16 range
    in a group over a packing (more than 8 tokens) gives the scaled
    packing's results (the fp32 entry computes it in EXACT arithmetic
    instead), and a non-finite output is counted."""
    from bonsai_b1 import synth
    m, k, n = 12, 3072, 1024
    x = synth.device_activations(m, k, 401)
    wa, wb, wc = (synth.device_packed_weights(n, k, 402 + i) for i in range(3))
    # two ops into one output: the second wins
    o = torch.empty((m, n), device="cuda")
    o2 = torch.empty((m, n), device="cuda")
    b1.linear_batch([(x, b1.device_weights(wa, k, n), o), (x, b1.device_weights(wb, k, n), o),
                     (x, b1.device_weights(wc, k, n), o2)])
    ref_b, ref_c = b1.linear(x, wb, n), b1.linear(x, wc, n)
    torch.cuda.synchronize()
    assert torch.equal(o, ref_b) and torch.equal(o2, ref_c)
    # the first output overwrites the input the second reads
    buf = torch.zeros((m, k), device="cuda")
    buf.copy_(x)
    b1.linear_batch([(buf, b1.device_weights(wa, k, n), buf[:, :n]),
                     (buf, b1.device_weights(wb, k, n), o)])
    x1 = x.clone()
    x1[:, :n] = b1.linear(x, wa, n)
    ref = b1.linear(x1, wb, n)
    torch.cuda.synchronize()
    assert torch.equal(buf[:, :n], x1[:, :n]) and torch.equal(o, ref)
    # beyond the fp16 range: row 1 x 1e5, row 2 all 3e38 (outputs overflow fp32)
    xb = x.clone()
    xb[1] *= 1e5
    xb[2] = 3.0e38
    ga, gb = torch.empty((m, n), device="cuda"), torch.empty((m, n), device="cuda")
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    b1.linear_batch([(xb, b1.device_weights(wa, k, n), ga), (xb, b1.device_weights(wb, k, n), gb)], nonfinite=nf)
    packed, rs = b1.pack_act_f16_scaled(xb)
    ya = b1.linear_packed_f16_scaled(packed, rs, wa, k, n, m)
    yb = b1.linear_packed_f16_scaled(packed, rs, wb, k, n, m)
    torch.cuda.synchronize()
    assert torch.equal(ga, ya) and torch.equal(gb, yb)
    bad = int((~torch.isfinite(ga)).sum() + (~torch.isfinite(gb)).sum())
    say(f"  non-finite outputs {bad}, counted {int(nf.item())}")
    assert bad > 0 and int(nf.item()) == bad
    assert bool(torch.isfinite(ga[[0, 1, 3, 11]]).all())


# ---------------------------------------------------------------- split-K --

SPLIT_CASES = [  # (m, k, n): shapes whose 128 x 512 tiles leave most CUs idle
    (256, 3072, 3072),    # C1: 12 tiles
    (512, 9216, 3072),    # Klein text stream FF-out: 24 tiles, long K
    (512, 3072, 9216),    # Klein text stream q/k/v
    (37, 15360, 384),     # one tile
    (200, 768, 600),
    (1000, 1152, 2100),
]


@pytest.mark.parametrize("m,k,n", SPLIT_CASES)
def test_split_k(torch, b1, m, k, n):
    """GEMMs split along K (work units of a tile and a K range, fp32 partial
    products summed in a fixed order by a second kernel): against the same
    GEMM unsplit, the difference is the summation order alone (<= 1e-5 of
    the output rms); against EXACT, the FAST bar; two runs are bit for bit
    the same; a padded, non-multiple-of-4 output stride is written only in
    its columns."""
    from bonsai_b1 import synth
    say(f"split-K ({m},{k},{n})")
    a = synth.device_activations(m, k, 45)
    w = synth.device_packed_weights(n, k, 46)
    y = b1.linear(a, w, n, mode="gemm")
    y2 = b1.linear(a, w, n, mode="gemm")
    yu = unsplit_linear(torch, b1, a, w, n, "gemm")
    ye = b1.linear(a, w, n, mode="exact")
    out = torch.full((m, n + 3), 7.0, device="cuda")
    b1.linear(a, w, n, out=out[:, :n], mode="gemm")
    torch.cuda.synchronize()
    assert torch.equal(y, y2), "split-K is deterministic"
    rms = float(yu.pow(2).mean().sqrt())
    d = float((y - yu).abs().max())
    say(f"  split vs unsplit max |diff| {d:.3e} (rms {rms:.3e}); identical: {bool(torch.equal(y, yu))}")
    assert d <= 1e-5 * rms
    assert_fast_close(y.cpu().numpy(), ye.cpu().numpy(), f"split-K {(m, k, n)} vs exact")
    assert torch.equal(out[:, :n], y)
    assert bool((out[:, n:] == 7.0).all()), "columns past out_dim untouched"


def test_split_k_counts_nonfinite(torch, b1):
    """The non-finite count comes from the summed outputs (the partials are
    not counted): an infinite activation makes its row's outputs non-finite
    in the split GEMM as in the unsplit one."""
    from bonsai_b1 import synth
    m, k, n = 256, 3072, 3072
    a = synth.device_activations(m, k, 47)
    a[5, 100] = float("inf")
    w = synth.device_packed_weights(n, k, 48)
    nf = torch.zeros(1, dtype=torch.int32, device="cuda")
    y = b1.linear(a, w, n, mode="gemm", nonfinite=nf)
    nfu = torch.zeros(1, dtype=torch.int32, device="cuda")
    ws = torch.empty(pack_area_bytes(m, k), dtype=torch.uint8, device="cuda")
    yu = b1.linear(a, w, n, mode="gemm", nonfinite=nfu, workspace=ws)
    torch.cuda.synchronize()
    bad = int((~torch.isfinite(y)).sum())
    say(f"  non-finite outputs {bad}, counted {int(nf.item())} split / {int(nfu.item())} unsplit")
    assert bad == n and int(nf.item()) == bad and int(nfu.item()) == int((~torch.isfinite(yu)).sum())


@pytest.mark.parametrize("m,k,n,splits", [(256, 3072, 3072, 8), (200, 768, 600, 2)])
def test_split_k_equals_per_range_composition(torch, b1, m, k, n, splits):
    """Bit for bit, on every one of several launches: the split GEMM equals
    the sum, in range order, of unsplit GEMMs over the K ranges (sliced
    activations and weights).  Regression test for an epilogue that
    rearranged accumulators across lanes before storing and intermittently
    stored stale values of one accumulator register in four lanes."""
    from bonsai_b1 import synth
    a = synth.device_activations(m, k, 45)
    w = synth.device_packed_weights(n, k, 46)
    wr = w.view(n, k // 32, 6)
    kr = k // splits
    ref = None
    for s in range(splits):
        ws_ = wr[:, s * kr // 32:(s + 1) * kr // 32, :].contiguous().view(-1)
        part = unsplit_linear(torch, b1, a[:, s * kr:(s + 1) * kr].contiguous(), ws_, n, "gemm")
        ref = part if ref is None else ref + part
    for run in range(6):
        y = b1.linear(a, w, n, mode="gemm")
        torch.cuda.synchronize()
        nbad = int((y != ref).sum())
        say(f"  run {run}: {nbad} elements differ")
        assert nbad == 0


@pytest.mark.parametrize("m,k,n", [(200, 384, 600), (256, 768, 1024)])
def test_one_tile_per_work_group_repeats(torch, b1, m, k, n):
    """Unsplit GEMMs with one output tile per work-group (the epilogue right
    after the last MFMAs, nothing in between): every launch gives the same
    bits and stays within the FAST bar of EXACT."""
    from bonsai_b1 import synth
    a = synth.device_activations(m, k, 49)
    w = synth.device_packed_weights(n, k, 50)
    ye = b1.linear(a, w, n, mode="exact")
    first = unsplit_linear(torch, b1, a, w, n, "gemm")
    for run in range(8):
        y = unsplit_linear(torch, b1, a, w, n, "gemm")
        torch.cuda.synchronize()
        assert torch.equal(y, first), f"launch {run}"
    assert_fast_close(first.cpu().numpy(), ye.cpu().numpy(), f"one tile per WG {(m, k, n)}")
