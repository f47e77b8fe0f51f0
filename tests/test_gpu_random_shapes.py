"""Seeded random shapes through the fp32 entry point in every mode, and
through its gate-residual epilogue, against the CPU oracle.

Bars (those of tests/test_gpu_parity.py and tests/test_gpu_epilogue.py):
  EXACT mode    : bit-identical to the oracle's scalar path
                  (src/b1_0_kernel.h:240-287).
  FAST modes    : auto, gemm and gemv against the oracle's AVX2 path
                  (src/b1_0_kernel.h:79-239): per element
                  |y - ref| / max(|ref|, rms(ref)) <= 1e-2, cosine >= 0.9999.
  gate-residual : bit for bit numpy's float32 residual + gate * y, y the
                  library's own linear in the same mode over a workspace
                  that holds the packing only (the GEMM then runs unsplit
                  along K, as the fused epilogue does).
  Columns past out_dim keep their sentinel in every mode.
The shapes are drawn so that every kernel choice of the library meets
ragged edges: M from 1 to 1300 (the small-M kernels up to several rounds of
tiles), K any multiple of 64 up to 4608 (K % 384 != 0 takes the
fused-conversion GEMM, K % 256 != 0 the fallback small-M kernel), N from 1
to 2600 (partial tiles, split-K and half-height tails where they apply),
and padded row strides.
"""
import random
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

TOL_REL = 1e-2
TOL_COS = 0.9999
EXACT_MAX_MACS = 5e8   # the scalar oracle's share of the test's time


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


def _draw(count, seed):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        band = rng.choice(["small", "mid", "large"])
        m = {"small": (1, 16), "mid": (17, 400), "large": (401, 1300)}[band]
        m = rng.randint(*m)
        k = 64 * rng.randint(1, 72)
        n = rng.randint(1, 2600)
        mode = rng.choice(["auto", "exact", "gemm"] + (["gemv"] if m <= 16 else []))
        if mode == "exact" and m * k * n > EXACT_MAX_MACS:
            mode = "auto"
        lda = k + 4 * rng.randint(1, 8) if rng.random() < 0.3 else None
        ldo = n + rng.randint(1, 16) if rng.random() < 0.3 else None
        cases.append((m, k, n, mode, lda, ldo))
    return cases


CASES = _draw(40, 20261202)


def _fast_close(y, ref):
    ref = np.asarray(ref, np.float64)
    y = np.asarray(y, np.float64)
    den = np.maximum(np.abs(ref), np.sqrt(np.mean(ref * ref)))
    rel = float(np.max(np.abs(y - ref) / den))
    cos = float((y.ravel() @ ref.ravel()) / (np.linalg.norm(y) * np.linalg.norm(ref)))
    return rel, cos


@pytest.mark.parametrize("m,k,n,mode,lda,ldo", CASES)
def test_random_shape(torch, b1, oracle, m, k, n, mode, lda, ldo):
    from bonsai_b1 import synth
    say(f"random shape ({m},{k},{n}) {mode} lda={lda} ldo={ldo}")
    act = synth.activations(m, k, m + 7 * k + 13 * n)
    raw = synth.packed_weights(n, k, m + k + n)
    if lda is None:
        a = torch.from_numpy(act).cuda()
    else:
        a = torch.zeros((m, lda), dtype=torch.float32)
        a[:, :k] = torch.from_numpy(act)
        a = a.cuda()[:, :k]
    w = torch.from_numpy(raw.ravel()).cuda()
    out = torch.full((m, ldo if ldo else n), 7.0, device="cuda")
    b1.linear(a, w, n, out=out[:, :n], mode=mode)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    if ldo:
        assert np.all(y[:, n:] == 7.0), "columns past out_dim untouched"
    y = y[:, :n]
    if mode == "exact":
        ref, _ = oracle.linear(act, raw, n, variant="scalar", nth=16, nthreads=16)
        say(f"  mismatching elements: {int((y.view(np.uint32) != ref.view(np.uint32)).sum())}")
        assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))
    else:
        ref, _ = oracle.linear(act, raw, n, variant="avx2", nth=16, nthreads=16)
        rel, cos = _fast_close(y, ref)
        say(f"  rel_to_rms={rel:.3e} cos={cos:.8f}")
        assert rel <= TOL_REL and cos >= TOL_COS

    # the gate-residual epilogue over the same linear
    ws = torch.empty((m * k * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256, dtype=torch.uint8,
                     device="cuda")
    yp = b1.linear(a, w, n, mode=mode, workspace=ws)
    g = torch.from_numpy(synth.activations(1, n, n + 5)[0]).cuda()
    pad = 3 if (m + n) % 2 else 0      # row stride of the residual: aligned or not
    res = torch.from_numpy(synth.activations(m, n + pad, m + 11)).cuda()[:, :n]
    got = b1.linear_epi(a, w, n, "gate_residual", gate=g, residual=res, mode=mode)
    torch.cuda.synchronize()
    want = res.cpu().numpy() + g.cpu().numpy()[None, :] * yp.cpu().numpy()   # float32 ops
    got = got.cpu().numpy()
    say(f"  gate-residual mismatching elements: {int((got.view(np.uint32) != want.view(np.uint32)).sum())}")
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


SWIGLU_TOL = 1e-6   # silu through the device exp and divide, a few fp32 ulp


def _draw_swiglu(count, seed):
    """Shapes for the SwiGLU epilogue: out_dim a multiple of 64 (gates and
    values, H = out_dim / 2 a multiple of 32)."""
    rng = random.Random(seed)
    cases = []
    for m, k, _, mode, lda, _ in _draw(count, seed):
        n = 64 * rng.randint(1, 40)
        if mode == "exact" and m * k * n > EXACT_MAX_MACS:
            mode = "auto"
        cases.append((m, k, n, mode, lda))
    return cases


@pytest.mark.parametrize("m,k,n,mode,lda", _draw_swiglu(16, 7))
def test_random_shape_swiglu(torch, b1, m, k, n, mode, lda):
    """out[:, j] = silu(y[:, j]) * y[:, H + j] against that formula in
    float64 on the library's own unsplit linear y, per element within
    1e-6 of the result; columns past H untouched."""
    from bonsai_b1 import synth
    say(f"random SwiGLU ({m},{k},{n}) {mode} lda={lda}")
    h = n // 2
    act = synth.activations(m, k, 3 * m + k + n)
    raw = synth.packed_weights(n, k, m + 5 * k + n)
    if lda is None:
        a = torch.from_numpy(act).cuda()
    else:
        a = torch.zeros((m, lda), dtype=torch.float32)
        a[:, :k] = torch.from_numpy(act)
        a = a.cuda()[:, :k]
    w = torch.from_numpy(raw.ravel()).cuda()
    ws = torch.empty((m * k * 2 + 255) // 256 * 256 + (m * 4 + 255) // 256 * 256, dtype=torch.uint8,
                     device="cuda")
    y = b1.linear(a, w, n, mode=mode, workspace=ws)
    out = torch.full((m, h + 4), 7.0, device="cuda")
    b1.linear_epi(a, w, n, "swiglu", out=out[:, :h], mode=mode)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert bool((got[:, h:] == 7.0).all()), "columns past H untouched"
    yy = y.cpu().numpy().astype(np.float64)
    ref = yy[:, :h] / (1.0 + np.exp(-yy[:, :h])) * yy[:, h:]
    bad = np.abs(got[:, :h] - ref) > SWIGLU_TOL * np.maximum(np.abs(ref), 1e-30) + 1e-30
    say(f"  {int(bad.sum())} elements beyond the bar")
    assert not bad.any()


def _batch_plan(seed):
    """A random sequence of linears over a pool of three fp32 activation
    matrices: some ops read a matrix that an earlier op of the same call
    wrote rows of (the cached packing must not outlive that write), some
    run back to back on one input with weights that are adjacent row
    ranges of one buffer and outputs adjacent column ranges of one matrix
    (q/k/v, run as one GEMM), small-M ops in a row on one input (grouped
    into one launch), K a multiple of 64 (the packed GEMM, the
    fused-conversion GEMM and the small-M kernels)."""
    rng = random.Random(seed)
    pool = []
    for _ in range(3):
        m = rng.choice([rng.randint(1, 16), rng.randint(17, 600)])
        k = rng.choice([384 * rng.randint(1, 8), 64 * rng.randint(1, 48)])
        pool.append((m, k))
    ops = []      # (input, [widths], out): out ("fresh",) or ("pool", q)
    last_in, last_written = None, None
    for _ in range(rng.randint(3, 9)):
        u = rng.random()
        if last_written is not None and u < 0.4:
            p = last_written            # read what an earlier op wrote
        elif last_in is not None and u < 0.7:
            p = last_in                 # the same input again (its packing reused)
        else:
            p = rng.randrange(3)
        last_in = p
        m, k = pool[p]
        widths = [rng.randint(1, 1500)]
        if rng.random() < 0.3:
            widths = [rng.randint(1, 700) for _ in range(3)]          # q/k/v
        elif m <= 16 and rng.random() < 0.5:
            widths = [rng.randint(1, 2000) for _ in range(rng.randint(2, 4))]   # a grouped run
        q = rng.randrange(3)
        if len(widths) == 1 and q != p and pool[q][0] >= m and pool[q][1] >= widths[0] and rng.random() < 0.5:
            ops.append((p, widths, ("pool", q)))
            last_written = q
        else:
            ops.append((p, widths, ("fresh",)))
    return pool, ops


@pytest.mark.parametrize("seed", range(12))
def test_random_batch(torch, b1, seed):
    """bonsai_b1_linear_batch over a random plan equals the same linears
    issued one by one in the same order, bit for bit: every output, and the
    pool matrices that ops wrote into."""
    from bonsai_b1 import synth
    pool, plan = _batch_plan(9000 + seed)
    mode = "exact" if seed % 4 == 3 else "auto"
    say(f"random batch seed={seed} mode={mode} pool={pool} ops={plan}")
    base = [synth.device_activations(m, k, 900 + 10 * seed + i) for i, (m, k) in enumerate(pool)]
    weights = []
    for j, (p, widths, _) in enumerate(plan):
        k = pool[p][1]
        big = synth.device_packed_weights(sum(widths), k, 950 + 20 * seed + j)
        weights.append(big.reshape(-1))     # rows of k / 32 * 6 bytes, sliced below

    def run(batched):
        mats = [x.clone() for x in base]
        outs, ops = [], []
        for (p, widths, dst), big in zip(plan, weights):
            m, k = pool[p]
            rs = k // 32 * 6
            if dst[0] == "pool":
                o = mats[dst[1]][:m, :widths[0]]
                parts = [o]
            else:
                o = torch.full((m, sum(widths) + 5), 7.0, device="cuda")
                outs.append(o)
                parts, c = [], 0
                for wd in widths:
                    parts.append(o[:, c:c + wd])
                    c += wd
            r = 0
            for wd, part in zip(widths, parts):
                wv = big[r * rs:(r + wd) * rs]
                if batched:
                    ops.append((mats[p], b1.device_weights(wv, k, wd), part))
                else:
                    b1.linear(mats[p], wv, wd, out=part, mode=mode)
                r += wd
        if batched:
            b1.linear_batch(ops, mode=mode)
        torch.cuda.synchronize()
        return mats, outs

    mats_b, outs_b = run(True)
    mats_s, outs_s = run(False)
    for i, (x, y) in enumerate(zip(outs_b, outs_s)):
        assert torch.equal(x, y), f"output {i}"
    for i, (x, y) in enumerate(zip(mats_b, mats_s)):
        assert torch.equal(x, y), f"pool matrix {i}"


def _draw_norm(count, seed):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        rows = rng.choice([rng.randint(1, 40), rng.randint(41, 3000)])
        h = 32 * rng.choice([rng.randint(1, 96), rng.randint(97, 384), rng.randint(385, 640)])
        pad = 4 * rng.randint(1, 8) if rng.random() < 0.4 else 0
        cases.append((rows, h, pad))
    return cases


@pytest.mark.parametrize("rows,h,pad", _draw_norm(14, 31))
def test_random_norm_mod(torch, b1, oracle, rows, h, pad):
    """LayerNorm + modulation over random row counts and lengths (rows held
    in registers up to 3072 and 12288 elements, read three times beyond),
    row strides padded or not: the fp32 form bit for bit the oracle's
    restatement of ggml_norm + modulation, the packed form its fp16
    packing."""
    say(f"random norm_mod rows={rows} h={h} pad={pad}")
    rng = np.random.default_rng(rows * 7 + h)
    x = (rng.standard_normal((rows, h + pad)) * 2 + 0.5).astype(np.float32)
    x[rows // 2, :] = -0.625                      # a constant row: var = 0
    sc = (rng.standard_normal(h) * 0.2).astype(np.float32)
    sh = (rng.standard_normal(h) * 0.2).astype(np.float32)
    xd = torch.from_numpy(x).cuda()[:, :h]
    scd, shd = torch.from_numpy(sc).cuda(), torch.from_numpy(sh).cuda()
    y = b1.norm_mod(xd, scd, shd, eps=1e-6)
    packed = b1.norm_mod(xd, scd, shd, eps=1e-6, packed=True)
    torch.cuda.synchronize()
    want = oracle.norm_mod(np.ascontiguousarray(x[:, :h]), sc, sh, eps=1e-6)
    got = y.cpu().numpy()
    nbad = int((got.view(np.uint32) != want.view(np.uint32)).sum())
    say(f"  {nbad} mismatching")
    assert nbad == 0
    words = packed.cpu().numpy().view(np.uint32).reshape(rows, h // 2)
    assert np.array_equal(words, oracle.pack_act_words(want))


@pytest.mark.parametrize("m,k,n", [(300, 16512, 640), (37, 24576, 520), (130, 16128, 700)])
def test_long_rows(torch, b1, oracle, m, k, n):
    """K past 16384 (the range-safe pack reads such rows twice instead of
    holding them in registers) and K just below it (four waves a row, eight
    units a lane), through the fp32 entry, one row scaled past the fp16
    range (it is packed scaled down by a power of two, its outputs scaled
    back): within the FAST bar of the oracle's AVX2 path, row by row."""
    from bonsai_b1 import synth
    say(f"long rows ({m},{k},{n})")
    act = synth.activations(m, k, k + n)
    act[m // 3] *= 1.0e5
    raw = synth.packed_weights(n, k, m + n)
    y = b1.linear(torch.from_numpy(act).cuda(), torch.from_numpy(raw.ravel()).cuda(), n)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    ref, _ = oracle.linear(act, raw, n, variant="avx2", nth=16, nthreads=16)
    for r in (m // 3, (m // 3 + 1) % m):
        rel, cos = _fast_close(y[r], ref[r])
        say(f"  row {r}: rel_to_rms={rel:.3e} cos={cos:.8f}")
        assert rel <= TOL_REL and cos >= TOL_COS
    keep = np.arange(m) != m // 3
    rel, cos = _fast_close(y[keep], ref[keep])
    say(f"  other rows: rel_to_rms={rel:.3e} cos={cos:.8f}")
    assert rel <= TOL_REL and cos >= TOL_COS


def _draw_producers(count, seed):
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        m = rng.choice([rng.randint(1, 40), rng.randint(41, 3000)])
        k1 = 32 * rng.randint(1, 128)
        k2 = 32 * rng.randint(1, 256)
        spad = 4 * rng.randint(0, 8)            # source row padding (16-byte rows)
        dpad = 32 * rng.randint(0, 3)           # packed row padding
        cases.append((m, k1, k2, spad, dpad))
    return cases


@pytest.mark.parametrize("m,k1,k2,spad,dpad", _draw_producers(12, 77))
def test_random_column_range_producers(torch, b1, m, k1, k2, spad, dpad):
    """The plain pack and the GELU pack writing adjacent column ranges of one
    packed matrix (row length k1 + k2 + dpad fp16 elements) from sources with
    padded rows: the range equals the packing of the fp32 concatenation
    [a1 | gelu_tanh(a2)] bit for bit, and the row padding keeps its
    sentinel."""
    from bonsai_b1 import synth
    say(f"random producers m={m} k1={k1} k2={k2} spad={spad} dpad={dpad}")
    a1 = synth.device_activations(m, k1 + spad, 5100 + m)[:, :k1]
    a2 = synth.device_activations(m, k2 + spad, 5200 + m)[:, :k2]
    ldp = k1 + k2 + dpad
    buf = torch.full((m * ldp * 2,), 0xAB, dtype=torch.uint8, device="cuda")
    b1.pack_act_f16(a1, packed=buf, ldp=ldp)
    b1.gelu_tanh_pack_f16(a2, packed=buf[k1 * 2:], ldp=ldp)
    want = b1.pack_act_f16(torch.cat([a1, b1.gelu_tanh(a2.contiguous())], 1))
    torch.cuda.synchronize()
    rows = buf.view(m, ldp * 2)
    assert torch.equal(rows[:, :(k1 + k2) * 2], want.view(m, (k1 + k2) * 2))
    assert bool((rows[:, (k1 + k2) * 2:] == 0xAB).all()), "row padding untouched"


def _draw_packed(count, seed):
    rng = random.Random(seed)
    return [(rng.choice([rng.randint(1, 16), rng.randint(17, 1300)]), 384 * rng.randint(1, 12),
             rng.randint(1, 2600)) for _ in range(count)]


@pytest.mark.parametrize("m,k,n", _draw_packed(16, 55))
def test_random_packed_entry(torch, b1, m, k, n):
    """bonsai_b1_linear_packed_f16 over pack_act_f16 of the activations gives
    the fp32 entry's outputs bit for bit: its FAST mode (M > 16 or K % 256
    == 0, the small-M kernel at M <= 16) or its GEMM mode (M <= 16 with K %
    256 != 0, where the packed entry keeps the GEMM tile), split along K
    alike."""
    from bonsai_b1 import synth
    mode = "auto" if (m > 16 or k % 256 == 0) else "gemm"
    say(f"random packed entry ({m},{k},{n}) vs fp32 {mode}")
    a = synth.device_activations(m, k, 5300 + m)
    w = synth.device_packed_weights(n, k, 5400 + n)
    ref = b1.linear(a, w, n, mode=mode)
    out = torch.full((m, n + 3), 7.0, device="cuda")
    b1.linear_packed_f16(b1.pack_act_f16(a), w, k, n, m, out=out[:, :n])
    torch.cuda.synchronize()
    assert torch.equal(out[:, :n], ref)
    assert bool((out[:, n:] == 7.0).all()), "columns past out_dim untouched"


@pytest.mark.parametrize("m,n", [(1, 3_800_000), (8, 3_800_000), (24, 3_800_000), (24, 7_600_000)])
def test_weights_past_2gib(torch, b1, oracle, m, n):
    """3.8 M weight rows at K = 3072: 2.19 GB of packed weights, past the
    31-bit range of a buffer resource.  M <= 16 then takes the small-M
    fallback kernel (64-bit addressing, no LDS staging), M = 24 the packed
    GEMM (32-bit weight offsets, below 4 GiB); 7.6 M rows (4.38 GB, past 32
    bits) take the GEMM that converts its activations tile by tile (64-bit
    addressing): within the FAST bar of the oracle's AVX2 path."""
    from bonsai_b1 import synth
    k = 3072
    say(f"weights past 2 GiB m={m} n={n}")
    act = synth.activations(m, k, 5500 + m)
    w = synth.device_packed_weights(n, k, 5501)
    assert w.numel() > 2 ** 31
    y = b1.linear(torch.from_numpy(act).cuda(), w, n)
    torch.cuda.synchronize()
    raw = w.cpu().numpy()
    del w
    torch.cuda.empty_cache()
    ref, _ = oracle.linear(act, raw, n, variant="avx2", nth=16, nthreads=16)
    rel, cos = _fast_close(y.cpu().numpy(), ref)
    say(f"  rel_to_rms={rel:.3e} cos={cos:.8f}")
    assert rel <= TOL_REL and cos >= TOL_COS


def test_activations_past_2gib(torch, b1, oracle):
    """180,000 tokens at K = 3072: 2.21 GB of fp32 activations (the
    range-safe pack reads them with 64-bit offsets; the packing, 1.1 GB,
    stays within the GEMM's 32-bit offsets), within the FAST bar of the
    oracle's AVX2 path; one token scaled past the fp16 range."""
    from bonsai_b1 import synth
    m, k, n = 180_000, 3072, 512
    say(f"activations past 2 GiB m={m}")
    act = synth.activations(m, k, 5600)
    act[m - 7] *= 1.0e5
    assert act.nbytes > 2 ** 31
    raw = synth.packed_weights(n, k, 5601)
    a = torch.from_numpy(act).cuda()
    y = b1.linear(a, torch.from_numpy(raw.ravel()).cuda(), n)
    torch.cuda.synchronize()
    y = y.cpu().numpy()
    del a
    torch.cuda.empty_cache()
    ref, _ = oracle.linear(act, raw, n, variant="avx2", nth=16, nthreads=16)
    # the scaled token against its own row (its outputs are 1e5 times the
    # others'), the other tokens together
    keep = np.arange(m) != m - 7
    rel, cos = _fast_close(y[keep], ref[keep])
    say(f"  other tokens: rel_to_rms={rel:.3e} cos={cos:.8f}")
    assert rel <= TOL_REL and cos >= TOL_COS
    rel, cos = _fast_close(y[m - 7], ref[m - 7])
    say(f"  scaled token: rel_to_rms={rel:.3e} cos={cos:.8f}")
    assert rel <= TOL_REL and cos >= TOL_COS


@pytest.mark.parametrize("seed", range(8))
def test_random_batch_epilogues(torch, b1, seed):
    """bonsai_b1_linear_batch_epi over a random sequence of plain,
    gate-residual and SwiGLU linears on two inputs (the packed GEMM, the
    small-M kernel or EXACT mode by shape and mode) equals the same linears
    issued one by one through the fp32 and epilogue entries, bit for bit."""
    from bonsai_b1 import synth
    rng = random.Random(9500 + seed)
    mode = "exact" if seed % 4 == 3 else "auto"
    inputs = []
    for i in range(2):
        m = rng.choice([rng.randint(1, 16), rng.randint(17, 700)])
        k = 384 * rng.randint(1, 8)
        inputs.append(synth.device_activations(m, k, 9600 + 10 * seed + i))
    plan = []
    for j in range(rng.randint(3, 8)):
        p = rng.randrange(2)
        kind = rng.choice(["none", "gate_residual", "swiglu"])
        n = 64 * rng.randint(1, 24) if kind == "swiglu" else rng.randint(1, 1500)
        plan.append((p, kind, n))
    say(f"random batch with epilogues seed={seed} mode={mode} "
        f"inputs={[tuple(x.shape) for x in inputs]} plan={plan}")
    ops, singles = [], []
    for j, (p, kind, n) in enumerate(plan):
        a = inputs[p]
        m, k = a.shape
        w = synth.device_packed_weights(n, k, 9700 + 20 * seed + j)
        cols = n // 2 if kind == "swiglu" else n
        out = torch.full((m, cols + 3), 7.0, device="cuda")[:, :cols]
        ref = torch.full((m, cols + 3), 7.0, device="cuda")[:, :cols]
        if kind == "gate_residual":
            g = synth.device_activations(1, n, 9800 + j)[0]
            r = synth.device_activations(m, n, 9900 + j)
            ops.append((a, b1.device_weights(w, k, n), out, ("gate_residual", g, r)))
            singles.append(lambda a=a, w=w, n=n, g=g, r=r, ref=ref:
                           b1.linear_epi(a, w, n, "gate_residual", gate=g, residual=r, out=ref, mode=mode))
        elif kind == "swiglu":
            ops.append((a, b1.device_weights(w, k, n), out, "swiglu"))
            singles.append(lambda a=a, w=w, n=n, ref=ref: b1.linear_epi(a, w, n, "swiglu", out=ref, mode=mode))
        else:
            ops.append((a, b1.device_weights(w, k, n), out))
            singles.append(lambda a=a, w=w, n=n, ref=ref: b1.linear(a, w, n, out=ref, mode=mode))
        plan[j] = (out, ref, w)
    b1.linear_batch(ops, mode=mode)
    for f in singles:
        f()
    torch.cuda.synchronize()
    for j, (out, ref, _) in enumerate(plan):
        full_o = out.as_strided((out.shape[0], out.shape[1] + 3), out.stride())
        full_r = ref.as_strided((ref.shape[0], ref.shape[1] + 3), ref.stride())
        assert torch.equal(full_o, full_r), f"op {j}"


@pytest.mark.parametrize("seed", range(6))
def test_random_quantize(torch, b1, oracle, seed):
    """The GPU writer over random shapes and magnitudes (per-row scales from
    1e-30 to 1e30, so fp16 scales that round to 0, to subnormals and to
    inf, blocks of one repeated magnitude, signed zeros): both reference
    writers' bytes (numpy's mean order and the left-to-right order), bit for
    bit."""
    rng = np.random.default_rng(9900 + seed)
    n = int(rng.integers(1, 2000))
    k = 32 * int(rng.integers(1, 200))
    say(f"random quantize seed={seed} n={n} k={k}")
    w = rng.standard_normal((n, k)).astype(np.float32)
    w *= (10.0 ** rng.uniform(-30, 30, (n, 1))).astype(np.float32)
    w[n // 2, :32] = np.float32(0.375) * np.sign(rng.standard_normal(32)).astype(np.float32)
    w[n // 3, :32] = -0.0
    dw = torch.from_numpy(w).cuda()
    for order in ("numpy", "sequential"):
        got = b1.quantize_f32(dw, order=order)
        torch.cuda.synchronize()
        want = oracle.pack(w, order=order)
        nbad = int((got.cpu().numpy() != want).sum())
        say(f"  {order}: {nbad} differing bytes")
        assert nbad == 0


@pytest.mark.parametrize("seed", range(8))
def test_random_gelu(torch, b1, seed):
    """GELU-tanh over random shapes (up to 3000 x 12000; the non-temporal
    form past 128 MB is checked at the C4 size in test_gpu_parity.py),
    padded row strides, out of place and in place: within 1e-6 max(1, |x|)
    of the float64 function, in place equal to out of place bit for bit,
    row padding untouched."""
    from oracle import b1_oracle
    rng = np.random.default_rng(9950 + seed)
    rows = int(rng.choice([rng.integers(1, 64), rng.integers(64, 3000)]))
    cols = 4 * int(rng.integers(1, 3000))
    px, py = 4 * int(rng.integers(0, 4)), 4 * int(rng.integers(0, 4))
    say(f"random GELU seed={seed} rows={rows} cols={cols} pads={px},{py}")
    x = (rng.standard_normal((rows, cols + px)) * 3).astype(np.float32)
    xd = torch.from_numpy(x).cuda()[:, :cols]
    yd = torch.full((rows, cols + py), 7.0, device="cuda")
    b1.gelu_tanh(xd, out=yd[:, :cols])
    inplace = torch.from_numpy(x).cuda()
    b1.gelu_tanh(inplace[:, :cols], out=inplace[:, :cols])
    torch.cuda.synchronize()
    y = yd.cpu().numpy()
    assert bool((y[:, cols:] == 7.0).all()), "row padding untouched"
    y = y[:, :cols]
    ref = b1_oracle.gelu_tanh_f64(x[:, :cols].astype(np.float64))
    err = float(np.max(np.abs(y - ref) / np.maximum(1.0, np.abs(x[:, :cols]))))
    say(f"  max err {err:.3e}")
    assert err <= 1e-6
    ip = inplace.cpu().numpy()
    assert np.array_equal(ip[:, :cols].view(np.uint32), y.view(np.uint32))
    assert np.array_equal(ip[:, cols:], x[:, cols:]), "padding of the in-place rows untouched"
