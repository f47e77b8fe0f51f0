"""GPU checks of the library under concurrent host callers.

The library keeps one workspace per (device, stream), hands it to a call
for the time the call takes to queue its kernels (a user count), replaces a
stream's buffer when a call needs a larger one, and, past 8 idle buffers on
a device, frees the least recently used one that no call holds (hipFree
waits for the kernels already queued on it).  Ten host threads, each on a
stream of its own, run linears whose workspace needs grow call by call, so
buffers are replaced and evicted while other threads' calls are in flight.
Bar: every output equals the same call made alone on one stream
beforehand, bit for bit (same kernels, same split along K).
The per-thread non-finite counter of the deferred callback is checked the
same way: each thread's count is its own.  The callback queues on
hipStreamPerThread, one handle value that names each thread's own stream:
its workspace must be kept per calling thread, or one thread's GEMM reads
another's packing (both tests below fail on a library that keyed it by the
handle alone).
"""
import sys
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

THREADS = 10


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


def _run_threads(fn):
    errors = []

    def wrap(t):
        try:
            fn(t)
        except BaseException as e:       # reported after the join
            errors.append((t, repr(e)))
    ths = [threading.Thread(target=wrap, args=(t,)) for t in range(THREADS)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    assert not errors, errors


def test_concurrent_callers_on_own_streams(torch, b1):
    from bonsai_b1 import synth
    k, n = 3072, 1536
    # per thread: fp32 linears of growing row counts (workspace: the fp16
    # packing, M K 2 bytes, plus row scales), a small-M call (no workspace)
    # and an EXACT one
    plans = []
    for t in range(THREADS):
        rows = [200 + 40 * t, 700 + 40 * t, 1500 + 40 * t, 8, 64]
        modes = ["auto", "auto", "auto", "auto", "exact"]
        acts = [synth.device_activations(m, k, 3000 + 10 * t + i) for i, m in enumerate(rows)]
        plans.append((rows, modes, acts))
    w = synth.device_packed_weights(n, k, 3999)
    refs = [[b1.linear(a, w, n, mode=md) for a, md in zip(acts, modes)] for rows, modes, acts in plans]
    torch.cuda.synchronize()
    outs = [[torch.full((a.shape[0], n), 7.0, device="cuda") for a in acts] for _, _, acts in plans]

    def work(t):
        s = torch.cuda.Stream()
        rows, modes, acts = plans[t]
        with torch.cuda.stream(s):
            for rep in range(3):
                for i, (a, md) in enumerate(zip(acts, modes)):
                    b1.linear(a, w, n, out=outs[t][i], mode=md, stream=s)
        s.synchronize()

    _run_threads(work)
    torch.cuda.synchronize()
    for t in range(THREADS):
        for i in range(len(plans[t][0])):
            assert torch.equal(outs[t][i], refs[t][i]), f"thread {t} call {i}"
    say(f"{THREADS} threads x {len(plans[0][0])} linears x 3 passes: all equal")


def test_concurrent_deferred_callbacks(torch, b1):
    """Each thread defers its callback checks (the callback then enqueues on
    the thread's own stream, hipStreamPerThread), runs three ops whose inputs
    hold t + 1 tokens with a NaN, and reads back exactly its own count: 3 (t
    + 1) out_dim; the outputs equal the library's AUTO linear."""
    import ctypes
    from bonsai_b1 import capi, synth
    k, n, m = 3072, 1024, 600
    W = b1.Weights(synth.packed_weights(n, k, 4001), k, n)
    acts = []
    for t in range(THREADS):
        a = synth.device_activations(m, k, 4100 + t)
        a[: t + 1, 5] = float("nan")
        acts.append(a)
    refs = [W.linear(a) for a in acts]
    torch.cuda.synchronize()
    ud = capi.B1LinearUserData(0x31423142, k, n)
    lib = b1.load()

    class T(ctypes.Structure):
        pass
    T._fields_ = [("ne", ctypes.c_int64 * 4), ("nb", ctypes.c_size_t * 4),
                  ("src", ctypes.POINTER(T) * 2), ("data", ctypes.c_void_p)]

    def node(x, o, keep):
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

    counts = [None] * THREADS
    outs = [[torch.full((m, n), 7.0, device="cuda") for _ in range(3)] for _ in range(THREADS)]
    torch.cuda.synchronize()

    def work(t):
        keep = []
        cnt = ctypes.c_int32(-1)
        assert lib.bonsai_b1_callback_defer(1) == capi.OK
        try:
            for o in outs[t]:
                lib.bonsai_b1_linear_f32_f32(ctypes.byref(node(acts[t], o, keep)), 0, 1, ctypes.byref(ud))
            st = lib.bonsai_b1_callback_finish(ctypes.byref(cnt))
            counts[t] = (st, cnt.value)
        finally:
            lib.bonsai_b1_callback_defer(0)

    _run_threads(work)
    torch.cuda.synchronize()
    for t in range(THREADS):
        assert counts[t] == (capi.ERR_NONFINITE, 3 * (t + 1) * n), (t, counts[t])
        for o in outs[t]:
            assert torch.equal(o.isnan(), refs[t].isnan()), t
            keep = ~refs[t].isnan()
            assert torch.equal(o[keep], refs[t][keep]), t
    W.free()


def test_per_thread_default_stream(torch, b1):
    """hipStreamPerThread, one handle value naming a different stream in
    each thread, passed to the fp32 entry by ten threads at once, four calls
    each with no synchronisation between them (each call packs its input
    into the library's workspace and splits the GEMM along K into partials
    there): every output bit for bit the same call made alone.  The library
    keeps such a stream's workspace per calling thread; shared by handle
    value, one thread's packing would be read by another's GEMM."""
    from bonsai_b1 import capi, synth
    m, k, n = 1024, 3072, 2048
    per_thread_stream = 2          # hipStreamPerThread
    w = synth.device_packed_weights(n, k, 4201)
    acts = [synth.device_activations(m, k, 4210 + t) for t in range(THREADS)]
    refs = [b1.linear(a, w, n) for a in acts]
    outs = [[torch.full((m, n), 7.0, device="cuda") for _ in range(4)] for _ in range(THREADS)]
    torch.cuda.synchronize()

    def work(t):
        for o in outs[t]:
            st = capi.linear_raw(acts[t].data_ptr(), k, w.data_ptr(), k, n, m, o.data_ptr(), n, "auto", 0,
                                 per_thread_stream)
            assert st == capi.OK, st

    _run_threads(work)
    torch.cuda.synchronize()
    for t in range(THREADS):
        for i, o in enumerate(outs[t]):
            assert torch.equal(o, refs[t]), f"thread {t} call {i}"
