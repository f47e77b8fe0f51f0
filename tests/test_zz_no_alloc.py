"""bonsai_b1_linear_f32_noalloc: the entry point that allocates nothing.

It runs the kernels of bonsai_b1_linear_f32 with their workspace (the fp16
packing and the split-K partials) in a static device array, so its outputs
must equal bonsai_b1_linear_f32's bit for bit.  Called through the C ABI
with raw device pointers.  Two calls in a row, the second smaller, so the
second runs over what the first left in the array; a call needing more
than the array holds is refused before anything is launched.
"""
import ctypes
import sys

import pytest

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as t
    assert t.cuda.is_available(), "GPU tests need the MI355X"
    return t


@pytest.fixture(scope="module")
def lib(torch):
    import bonsai_b1
    return bonsai_b1.load()


def _call(lib, torch, fn, a, w, n, out, mode):
    from bonsai_b1 import capi
    m, k = a.shape
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    return getattr(lib, fn)(a.data_ptr(), a.stride(0), w.data_ptr(), k, n, m, out.data_ptr(), out.stride(0),
                            capi.MODES[mode], None, stream)


# (M, K, N, mode): the first needs the packing plus split-K partials
# (256 x 3072 x 3072 splits K eight ways on 256 CUs: 1.5 MB + 25.2 MB), the
# second a smaller packing over the first one's leftovers, then small-M
# and EXACT calls that need none.
SEQUENCE = [(256, 3072, 3072, "auto"), (160, 768, 600, "gemm"), (8, 3072, 4096, "auto"), (5, 256, 40, "exact")]


def test_noalloc_matches_linear_f32(torch, lib):
    from bonsai_b1 import capi, synth
    for i, (m, k, n, mode) in enumerate(SEQUENCE):
        say(f"no-alloc call {i}: M={m} K={k} N={n} mode={mode}")
        need = capi.workspace_bytes(m, k, n, mode)
        assert need <= capi.NOALLOC_SCRATCH_BYTES
        a = synth.device_activations(m, k, 500 + i)
        w = synth.device_packed_weights(n, k, 600 + i)
        ref = torch.full((m, n), 3.0, device="cuda")
        got = torch.full((m, n + 8), 7.0, device="cuda")[:, :n]
        assert _call(lib, torch, "bonsai_b1_linear_f32", a, w, n, ref, mode) == capi.OK
        assert _call(lib, torch, "bonsai_b1_linear_f32_noalloc", a, w, n, got, mode) == capi.OK
        torch.cuda.synchronize()
        say(f"  workspace {need} B; max |diff| {float((got - ref).abs().max()):.3e}")
        assert torch.equal(got, ref), f"call {i} differs from bonsai_b1_linear_f32"


def test_noalloc_refuses_oversized_call(torch, lib):
    """4608 x 12288 activations need a 113 MB packing: refused with
    ERR_SCRATCH, nothing written."""
    from bonsai_b1 import capi, synth
    m, k, n = 4608, 12288, 64
    assert capi.workspace_bytes(m, k, n, "auto") > capi.NOALLOC_SCRATCH_BYTES
    a = torch.zeros((m, k), device="cuda")
    w = synth.device_packed_weights(n, k, 7)
    out = torch.full((m, n), 5.0, device="cuda")
    say("no-alloc oversized call")
    assert _call(lib, torch, "bonsai_b1_linear_f32_noalloc", a, w, n, out, "auto") == capi.ERR_SCRATCH
    torch.cuda.synchronize()
    assert bool((out == 5.0).all())
    # a call that fails its argument checks is ERR_ARG whatever its size
    assert lib.bonsai_b1_linear_f32_noalloc(a.data_ptr(), k, w.data_ptr(), k + 1, n, m, out.data_ptr(), n,
                                            0, None, None) == capi.ERR_ARG


def test_noalloc_takes_unaligned_call_of_any_size(torch, lib):
    """The same oversized shape over activations that are not 16-byte
    aligned (row stride K + 1): such a call runs EXACT mode, which needs no
    workspace, so it is accepted and equals bonsai_b1_linear_f32 bit for
    bit."""
    from bonsai_b1 import capi, synth
    m, k, n = 4608, 12288, 64
    buf = torch.empty((m, k + 1), device="cuda")
    buf[:, 1:] = synth.device_activations(m, k, 8)
    a = buf[:, 1:]
    w = synth.device_packed_weights(n, k, 9)
    ref = torch.full((m, n), 3.0, device="cuda")
    got = torch.full((m, n), 5.0, device="cuda")
    say("no-alloc unaligned call")
    assert _call(lib, torch, "bonsai_b1_linear_f32", a, w, n, ref, "auto") == capi.OK
    assert _call(lib, torch, "bonsai_b1_linear_f32_noalloc", a, w, n, got, "auto") == capi.OK
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_noalloc_under_graph_capture(torch, lib):
    """Captured on a stream the library has never seen (so it owns no
    workspace for it, and a capture cannot allocate one), the no-alloc entry
    still runs the packed GEMM, split along K (256 x 3072 x 3072: 26.7 MB of
    packing and partials); every replay equals the eager result, with other
    no-alloc calls between the replays."""
    from bonsai_b1 import capi, synth
    m, k, n = 256, 3072, 3072
    assert capi.workspace_bytes(m, k, n, "auto") <= capi.NOALLOC_SCRATCH_BYTES
    a = synth.device_activations(m, k, 71)
    w = synth.device_packed_weights(n, k, 72)
    ref = torch.empty((m, n), device="cuda")
    assert _call(lib, torch, "bonsai_b1_linear_f32", a, w, n, ref, "auto") == capi.OK
    y = torch.empty((m, n), device="cuda")
    other = torch.empty((64, 600), device="cuda")
    a2 = synth.device_activations(64, 768, 73)
    w2 = synth.device_packed_weights(600, 768, 74)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    say("no-alloc graph capture")
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            assert _call(lib, torch, "bonsai_b1_linear_f32_noalloc", a, w, n, y, "auto") == capi.OK
    torch.cuda.synchronize()
    for i in range(3):
        y.fill_(float(i + 1))
        assert _call(lib, torch, "bonsai_b1_linear_f32_noalloc", a2, w2, 600, other, "gemm") == capi.OK
        g.replay()
        torch.cuda.synchronize()
        say(f"  replay {i}: max |diff| {float((y - ref).abs().max()):.3e}")
        assert torch.equal(y, ref), f"replay {i}"
