#!/usr/bin/env python3
"""Benchmark of the gfx950 B1_0 1-bit linear (one MI355X).

Default workload: the B1_0 GEMM at M=4096 (tokens), K=3072, N=12288 on
synthetic data (activations N(0,1) fp32, random sign words, fp16 scales
U[0.005, 0.05]), inputs resident in HBM before timing.  One step = one
B1_0 linear over that batch (the range-safe fp16 pack pass + the MFMA GEMM).
Before any timing the shader clock is settled by running the step for a
fixed wall time (--settle-s), and read while the GPU is still busy.  Prints
ONE JSON line with the metric, the MFMA roofline of the GEMM kernel (and
the pack pass timed alone), the small-M GEMV bandwidth (M=8, K=3072,
N=18432, weight copies rotated past the 256 MB Infinity Cache), the other
config shapes (C1, C3, C4, the C5 38-block step) and the CPU baseline (the
oracle's restatement of the reference AVX2 path on this host, at the host's
thread share and at the reference's default of 4 threads).

  python bench.py [--steps K] [--warmup W] [--settle-s S] [--gpus 1] [--all] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path[:0] = [str(ROOT), str(ROOT / "bonsai.cpp_amd")]

PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16/bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3    # MI355X fp32 (vector and matrix)
HEADLINE = (4096, 3072, 12288)
GEMV = (8, 3072, 18432)
MALL_BYTES = 256 << 20
TRAFFIC_PROFILE = "b1_gemm_kernel_m4096_k3072_n12288_traffic"


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def time_launches(torch, fn, steps, warmup):
    """Average GPU time per call (ms) from events on the launch stream, plus
    the host wall time of the timed region."""
    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(s)
    for i in range(steps):
        fn(i)
    e1.record(s)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / steps, wall


_BENCH_LIB = None


def read_floor(torch, bufs, nbytes, steps, warmup):
    """The HBM read floor of a small-M leg: a kernel that only reads
    `nbytes` of each buffer (16 bytes a lane, four loads in flight, the
    result folded into a word that is never stored; lib/libb1bench.so),
    replayed as a HIP graph over the same rotated copies as the leg.  The
    best of three grid shapes; per-launch time, as the leg reports it."""
    global _BENCH_LIB
    import ctypes
    if _BENCH_LIB is None:
        _BENCH_LIB = ctypes.CDLL(str(ROOT / "bonsai.cpp_amd" / "lib" / "libb1bench.so"))
        _BENCH_LIB.b1bench_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int,
                                            ctypes.c_int, ctypes.c_void_p]
        _BENCH_LIB.b1bench_read.restype = ctypes.c_int
    best = None
    for nwg, block in ((1024, 512), (2048, 256), (512, 1024)):
        sink = torch.zeros(nwg, dtype=torch.int32, device="cuda")

        def call(c):
            st = torch.cuda.current_stream().cuda_stream
            rc = _BENCH_LIB.b1bench_read(ctypes.c_void_p(bufs[c].data_ptr()), nbytes, ctypes.c_void_p(sink.data_ptr()),
                                         nwg, block, ctypes.c_void_p(st))
            assert rc == 0, rc
        call(0)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for c in range(len(bufs)):
                call(c)
        reps = max(1, steps // len(bufs))
        ms, _ = time_launches(torch, lambda i: graph.replay(), reps, max(1, warmup // len(bufs)))
        ms /= len(bufs)
        if best is None or ms < best[0]:
            best = (ms, nwg, block)
    ms, nwg, block = best
    return {"us": ms * 1e3, "GBps": nbytes / (ms * 1e-3) / 1e9, "frac_hbm": nbytes / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS,
            "grid": [nwg, block], "bytes": nbytes}


def bench_gemm(torch, b1, synth, m, k, n, steps, warmup, mode="auto", inputs=None):
    """The whole op from fp32 activations, bonsai_b1_linear_f32 with the
    library's workspace: the range-safe pack pass, then the GEMM (split
    along K where the shape asks for it)."""
    if inputs is None:
        inputs = (synth.device_activations(m, k, 1), synth.device_packed_weights(n, k, 2))
    a, w = inputs
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    ms, wall = time_launches(torch, lambda i: b1.linear(a, w, n, out=y, mode=mode), steps, warmup)
    flop = 2.0 * m * n * k
    return {"shape": [m, k, n], "ms": ms, "tflops": flop / (ms * 1e-3) / 1e12,
            "frac": flop / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, "wall_s": wall, "inputs": (a, w)}


# (name, (M, K, N), epilogue, tile): the shapes the 16x16 tile kernels run,
# 144 x 384 at M = 4608 and 128 x 384 at the Klein image stream's M = 4096
TILES16_SHAPES = [("c3_qkv", (4608, 3072, 9216), "none", "144x384"), ("c3_out", (4608, 3072, 3072), "none", "144x384"),
                  ("c4_up", (4608, 3072, 12288), "none", "144x384"), ("c4_down", (4608, 12288, 3072), "none", "144x384"),
                  ("c5_linear2", (4608, 15360, 3072), "gate_residual", "144x384"),
                  ("klein_single_linear1", (4608, 3072, 27648), "none", "144x384"),
                  ("klein_img_qkv", (4096, 3072, 9216), "none", "128x384"),
                  ("klein_img_out", (4096, 3072, 3072), "none", "128x384"),
                  ("klein_img_ff_in", (4096, 3072, 18432), "none", "128x384"),
                  ("klein_img_ff_out", (4096, 9216, 3072), "none", "128x384")]


def bench_tiles16(torch, b1, synth, steps, warmup):
    """The 16x16 tile GEMMs (b1_gemm16_kernel, 144 x 384 and 128 x 384) alone
    at the Flux and Klein shapes they run: packed activations made once,
    then the packed entry (range-safe row scales, or the gate-residual
    epilogue for C5's linear2) timed with HIP events on its launch
    stream."""
    out = {}
    for name, (m, k, n), epi, tile in TILES16_SHAPES:
        a = synth.device_activations(m, k, 21)
        w = synth.device_packed_weights(n, k, 22)
        pa, rs = b1.pack_act_f16_scaled(a)
        y = torch.empty((m, n), device="cuda")
        if epi == "gate_residual":
            g = 0.1 * torch.randn(n, device="cuda")
            r = torch.randn((m, n), device="cuda")
            fn = lambda i: b1.linear_packed_f16_epi(pa, w, k, n, m, "gate_residual", gate=g, residual=r, out=y)
        else:
            fn = lambda i: b1.linear_packed_f16_scaled(pa, rs, w, k, n, m, out=y)
        ms, _ = time_launches(torch, fn, steps, warmup)
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        out[name] = {"shape": [m, k, n], "epilogue": epi, "tile": tile, "kernel_us": round(ms * 1e3, 2),
                     "tflops": round(tf, 1), "frac": round(tf / PEAK_FP16_TFLOPS, 4)}
        log(f"[bench] {tile} tiles {name} {(m, k, n)} {epi}: {ms * 1e3:.1f} us {tf:.1f} TFLOP/s "
            f"({100 * tf / PEAK_FP16_TFLOPS:.1f}% of peak)")
        del a, w, pa, rs, y
    return out


def bench_step_kernels(torch, b1, a, w, n, steps, warmup):
    """The two kernels of the step, each timed alone with HIP events on its
    launch stream: the GEMM kernel over packed activations
    (bonsai_b1_linear_packed_f16_scaled: b1_gemm_kernel alone at an unsplit
    shape) and the range-safe pack pass (bonsai_b1_pack_act_f16_scaled:
    b1_pack_rows_kernel alone).  Returns (gemm ms, pack ms)."""
    m, k = a.shape
    packed, rs = b1.pack_act_f16_scaled(a)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    kern_ms, _ = time_launches(torch, lambda i: b1.linear_packed_f16_scaled(packed, rs, w, k, n, m, out=y), steps,
                               warmup)
    pack_ms, _ = time_launches(torch, lambda i: b1.pack_act_f16_scaled(a, packed=packed, row_scale=rs), steps,
                               warmup)
    return kern_ms, pack_ms


def committed_traffic(name):
    """HBM bytes per launch of a kernel, from the committed rocprofv3 PMC
    summary profiles/<name>.md (FETCH_SIZE and WRITE_SIZE per dispatch,
    scaled by the plain-copy calibration written there); None if absent."""
    f = ROOT / "profiles" / f"{name}.md"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(line.split(":", 1)[1].strip())
    return None


def graph_ms(torch, record, reps=3):
    """One eager pass of record() (a sequence of library calls on the current
    stream), then the same calls captured into a HIP graph and replayed;
    returns the GPU time per replay (ms) from events around the replays."""
    record()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        record()
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


def bench_mlp(torch, b1, synth):
    """Flux MLP at 1024x1024 (4608 tokens): up-projection 3072 -> 12288,
    GELU-tanh, down-projection 12288 -> 3072; each part and the chain, plus
    the chain with GELU fused into the fp16 packing of the down-projection's
    input, and with GELU in the up-projection's epilogue writing that
    packing directly."""
    m, k, h = 4608, 3072, 12288
    a = synth.device_activations(m, k, 11)
    wu = synth.device_packed_weights(h, k, 12)
    wd = synth.device_packed_weights(k, h, 13)
    y1 = torch.empty((m, h), device="cuda")
    g = torch.empty((m, h), device="cuda")
    y2 = torch.empty((m, k), device="cuda")
    ws = torch.empty(max(b1.workspace_bytes(m, k, h), b1.workspace_bytes(m, h, k)), dtype=torch.uint8,
                     device="cuda")
    packed = torch.empty(m * h * 2, dtype=torch.uint8, device="cuda")

    def up():
        b1.linear(a, wu, h, out=y1, workspace=ws)

    def gelu():
        b1.gelu_tanh(y1, out=g)

    def down():
        b1.linear(g, wd, k, out=y2, workspace=ws)

    def fused():
        up()
        b1.gelu_tanh_pack_f16(y1, packed=packed)
        b1.linear_packed_f16(packed, wd, h, k, m, out=y2)

    r = {name: graph_ms(torch, lambda f=f: [f() for _ in range(4)]) / 4
         for name, f in (("up", up), ("gelu", gelu), ("down", down))}
    r["chain"] = graph_ms(torch, lambda: (up(), gelu(), down()))
    r["chain_fused_gelu"] = graph_ms(torch, fused)
    pa = torch.empty(m * k * 2, dtype=torch.uint8, device="cuda")

    def epilogue():
        # GELU in the up-projection's epilogue, written as the packed input
        # of the down-projection
        b1.pack_act_f16(a, packed=pa)
        b1.linear_packed_f16_to_packed(pa, wu, k, h, m, 0, "gelu_tanh", packed_out=packed)
        b1.linear_packed_f16(packed, wd, h, k, m, out=y2)

    r["chain_epilogue_gelu"] = graph_ms(torch, epilogue)
    flop = 2.0 * m * k * h * 2
    r["chain_tflops"] = flop / (r["chain"] * 1e-3) / 1e12
    r["chain_fused_tflops"] = flop / (r["chain_fused_gelu"] * 1e-3) / 1e12
    r["chain_epilogue_tflops"] = flop / (r["chain_epilogue_gelu"] * 1e-3) / 1e12
    r["gelu_GBps"] = m * h * 8 / (r["gelu"] * 1e-3) / 1e9
    return r


def bench_ff_epilogues(torch, b1, synth):
    """The double-block feed-forward of the reference graph at 64x64 latents
    (src/diffuser_graph.cpp:450-460, 4096 image tokens): FF-in 3072 ->
    2 x 9216, SwiGLU, FF-out 9216 -> 3072, gate-residual add into h.  Once
    with the element-wise steps as separate torch passes over the linears'
    fp32 outputs, once with both fused into the GEMM epilogues, and once
    with FF-in's SwiGLU epilogue writing FF-out's packed fp16 input."""
    m, d, hid = 4096, 3072, 9216
    x = synth.device_activations(m, d, 21)
    w_in = synth.device_packed_weights(2 * hid, d, 22)
    w_out = synth.device_packed_weights(d, hid, 23)
    gate = torch.randn(d, device="cuda")
    h = torch.randn((m, d), device="cuda")
    y1 = torch.empty((m, 2 * hid), device="cuda")
    act = torch.empty((m, hid), device="cuda")
    y2 = torch.empty((m, d), device="cuda")
    ws = torch.empty(max(b1.workspace_bytes(m, d, 2 * hid), b1.workspace_bytes(m, hid, d)), dtype=torch.uint8,
                     device="cuda")

    def separate():
        b1.linear(x, w_in, 2 * hid, out=y1, workspace=ws)
        torch.mul(torch.nn.functional.silu(y1[:, :hid]), y1[:, hid:], out=act)
        b1.linear(act, w_out, d, out=y2, workspace=ws)
        h.add_(gate * y2)

    def fused():
        b1.linear_epi(x, w_in, 2 * hid, "swiglu", out=act, workspace=ws)
        b1.linear_epi(act, w_out, d, "gate_residual", gate=gate, residual=h, out=h, workspace=ws)

    px = torch.empty(m * d * 2, dtype=torch.uint8, device="cuda")
    pk = torch.empty(m * hid * 2, dtype=torch.uint8, device="cuda")

    def packed_out():
        # SwiGLU in FF-in's epilogue written as FF-out's packed input
        b1.pack_act_f16(x, packed=px)
        b1.linear_packed_f16_to_packed(px, w_in, d, 2 * hid, m, 0, "swiglu", packed_out=pk)
        b1.linear_packed_f16_epi(pk, w_out, hid, d, m, "gate_residual", gate=gate, residual=h, out=h)

    r = {"separate": graph_ms(torch, separate), "fused": graph_ms(torch, fused),
         "fused_packed_out": graph_ms(torch, packed_out)}
    flop = 2.0 * m * d * (2 * hid) + 2.0 * m * hid * d
    r["fused_tflops"] = flop / (r["fused"] * 1e-3) / 1e12
    r["fused_packed_out_tflops"] = flop / (r["fused_packed_out"] * 1e-3) / 1e12
    return r


def bench_norm_mod(torch, b1, synth):
    """LayerNorm + modulation of 4096 image tokens x 3072 straight into the
    packed fp16 activations, against the same values through the separate
    fp32 producer and the pack pass."""
    m, d = 4096, 3072
    x = synth.device_activations(m, d, 31)
    sc = torch.randn(d, device="cuda") * 0.1
    sh = torch.randn(d, device="cuda") * 0.1
    y = torch.empty((m, d), device="cuda")
    packed = torch.empty(m * d * 2, dtype=torch.uint8, device="cuda")
    r = {"fused_pack": graph_ms(torch, lambda: [b1.norm_mod(x, sc, sh, packed=packed) for _ in range(8)]) / 8,
         "fp32_then_pack": graph_ms(torch, lambda: [(b1.norm_mod(x, sc, sh, out=y), b1.pack_act_f16(y, packed=packed))
                                                    for _ in range(8)]) / 8}
    r["fused_GBps"] = m * d * 6 / (r["fused_pack"] * 1e-3) / 1e9
    return r


def bench_single_stream_step(torch, b1, synth, blocks=38):
    """One diffusion step's worth of the Flux single-stream block linears,
    back to back on one stream: per block, linear1 4608 x 3072 -> 21504 and
    linear2 4608 x 15360 -> 3072, every block with its own resident weights
    (807 MB packed).  Activations are synthetic stand-ins of the right
    shapes.  Two dispatches: the fp32 op per linear, and the fp16-packed
    path (pack + packed GEMM)."""
    m, k1, n1, k2, n2 = 4608, 3072, 21504, 15360, 3072
    w1 = [synth.device_packed_weights(n1, k1, 300 + i) for i in range(blocks)]
    w2 = [synth.device_packed_weights(n2, k2, 400 + i) for i in range(blocks)]
    a1 = synth.device_activations(m, k1, 14)
    a2 = synth.device_activations(m, k2, 15)
    o1 = torch.empty((m, n1), device="cuda")
    o2 = torch.empty((m, n2), device="cuda")
    ws = torch.empty(max(b1.workspace_bytes(m, k1, n1), b1.workspace_bytes(m, k2, n2)), dtype=torch.uint8,
                     device="cuda")
    p1 = torch.empty(m * k1 * 2, dtype=torch.uint8, device="cuda")
    p2 = torch.empty(m * k2 * 2, dtype=torch.uint8, device="cuda")

    def step():
        for i in range(blocks):
            b1.linear(a1, w1[i], n1, out=o1, workspace=ws)
            b1.linear(a2, w2[i], n2, out=o2, workspace=ws)

    # inputs already in the packed fp16 layout, as the fused producers
    # (norm_mod_pack_f16 for linear1, gelu_tanh_pack_f16 for linear2's MLP
    # part) write them: the step is then the GEMMs alone
    b1.pack_act_f16(a1, packed=p1)
    b1.pack_act_f16(a2, packed=p2)

    def step_packed():
        for i in range(blocks):
            b1.linear_packed_f16(p1, w1[i], k1, n1, m, out=o1)
            b1.linear_packed_f16(p2, w2[i], k2, n2, m, out=o2)

    ms = graph_ms(torch, step, reps=2)
    flop = 2.0 * m * (k1 * n1 + k2 * n2) * blocks
    r = {"blocks": blocks, "ms_per_step": ms, "tflops": flop / (ms * 1e-3) / 1e12,
         "packed_weight_bytes": sum(w.numel() for w in w1 + w2)}
    r["ms_per_step_packed_inputs"] = graph_ms(torch, step_packed, reps=2)
    r["tflops_packed_inputs"] = flop / (r["ms_per_step_packed_inputs"] * 1e-3) / 1e12
    del w1, w2
    return r


def bench_c5_block_chain(torch, b1, synth, blocks=38, producer_form=False):
    """The C5 step: 38 single-stream blocks as a chain of this library's
    kernels, attention aside (src/diffuser_graph.cpp:477-538 in shape),
    each block with its own resident weights (807 MB packed).  Per block:
    LayerNorm + modulation written as packed fp16, linear1 3072 -> 21504
    with its epilogue writing q/k/v as fp32 and GELU-tanh(MLP) straight into
    columns 3072-15359 of linear2's packed input, the q columns (standing in
    for the attention output) packed into columns 0-3071, and linear2 15360
    -> 3072 with the gate-residual epilogue updating the residual stream in
    place; block i + 1 reads what block i wrote.  Timed as a HIP graph
    replay.  Also timed: the 76 GEMMs alone over inputs already packed (the
    step's GEMM work), and, with producer_form, the chain with GELU(MLP) made
    by a separate producer pass over linear1's fp32 output."""
    m, h, n1, k2 = 4608, 3072, 21504, 15360
    w1 = [synth.device_packed_weights(n1, h, 500 + i) for i in range(blocks)]
    w2 = [synth.device_packed_weights(h, k2, 600 + i) for i in range(blocks)]
    g = torch.Generator(device="cuda").manual_seed(5)
    scale = [0.1 * torch.randn(h, device="cuda", generator=g) for _ in range(blocks)]
    shift = [0.1 * torch.randn(h, device="cuda", generator=g) for _ in range(blocks)]
    gate = [0.05 * torch.randn(h, device="cuda", generator=g) for _ in range(blocks)]
    x = synth.device_activations(m, h, 17)
    p1 = torch.empty(m * h * 2, dtype=torch.uint8, device="cuda")
    y1 = torch.empty((m, n1), device="cuda")
    p2 = torch.empty(m * k2 * 2, dtype=torch.uint8, device="cuda")

    def step_producers():
        for i in range(blocks):
            b1.norm_mod(x, scale[i], shift[i], packed=p1)
            b1.linear_packed_f16(p1, w1[i], h, n1, m, out=y1)
            b1.pack_act_f16(y1[:, :h], packed=p2, ldp=k2)
            b1.gelu_tanh_pack_f16(y1[:, 3 * h:], packed=p2[h * 2:], ldp=k2)
            b1.linear_packed_f16_epi(p2, w2[i], k2, h, m, "gate_residual", gate=gate[i], residual=x, out=x)

    def step():
        for i in range(blocks):
            b1.norm_mod(x, scale[i], shift[i], packed=p1)
            b1.linear_packed_f16_to_packed(p1, w1[i], h, n1, m, 3 * h, "gelu_tanh", out=y1[:, :3 * h],
                                           packed_out=p2[h * 2:], ldp=k2)
            b1.pack_act_f16(y1[:, :h], packed=p2, ldp=k2)
            b1.linear_packed_f16_epi(p2, w2[i], k2, h, m, "gate_residual", gate=gate[i], residual=x, out=x)

    o2 = torch.empty((m, h), device="cuda")

    def step_gemms():
        for i in range(blocks):
            b1.linear_packed_f16(p1, w1[i], h, n1, m, out=y1)
            b1.linear_packed_f16(p2, w2[i], k2, h, m, out=o2)

    flop = 2.0 * m * (h * n1 + k2 * h) * blocks
    ms = graph_ms(torch, step, reps=2)
    finite = bool(torch.isfinite(x).all())
    ms_gemms = graph_ms(torch, step_gemms, reps=2)
    r = {"blocks": blocks, "ms_per_step": ms, "gemm_tflops": flop / (ms * 1e-3) / 1e12,
         "frac": flop / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, "kernels_per_block": 4,
         "ms_per_step_gemms_only": ms_gemms, "gemms_only_tflops": flop / (ms_gemms * 1e-3) / 1e12,
         "gemms_only_frac": flop / (ms_gemms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS,
         "packed_weight_bytes": sum(t.numel() for t in w1 + w2)}
    if producer_form:
        r["ms_per_step_producer_form"] = graph_ms(torch, step_producers, reps=2)
        finite = finite and bool(torch.isfinite(x).all())
    r["residual_finite"] = finite
    del w1, w2
    return r


def bench_c4_mlp(torch, b1, synth, reps=4):
    """C4 between its GEMMs: the standalone GELU-tanh over the up-projection's
    fp32 output (4608 x 12288, into a separate buffer), and the C4
    chain in its fused form (pack, up-projection with GELU in its epilogue
    written as the down-projection's packed input, down-projection), each
    captured into a HIP graph and replayed."""
    out = {}
    m, k, hid = 4608, 3072, 12288
    a = synth.device_activations(m, k, 11)
    wu = synth.device_packed_weights(hid, k, 12)
    wd = synth.device_packed_weights(k, hid, 13)
    y1 = torch.empty((m, hid), device="cuda")
    g = torch.empty((m, hid), device="cuda")
    pa = torch.empty(m * k * 2, dtype=torch.uint8, device="cuda")
    rs = torch.empty(m, dtype=torch.float32, device="cuda")
    ph = torch.empty(m * hid * 2, dtype=torch.uint8, device="cuda")
    y2 = torch.empty((m, k), device="cuda")
    b1.linear(a, wu, hid, out=y1)
    gelu_ms = graph_ms(torch, lambda: [b1.gelu_tanh(y1, out=g) for _ in range(reps)]) / reps

    def chain():
        b1.pack_act_f16_scaled(a, packed=pa, row_scale=rs)
        b1.linear_packed_f16_to_packed(pa, wu, k, hid, m, 0, "gelu_tanh", packed_out=ph)
        b1.linear_packed_f16(ph, wd, hid, k, m, out=y2)
    chain_ms = graph_ms(torch, chain)
    flop = 2.0 * m * k * hid * 2
    out["c4_gelu"] = {"shape": [m, hid], "us": round(gelu_ms * 1e3, 2),
                      "GBps": round(m * hid * 8 / (gelu_ms * 1e-3) / 1e9, 1),
                      "frac_hbm": round(m * hid * 8 / (gelu_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
    out["c4_chain"] = {"shape": [m, k, hid], "us": round(chain_ms * 1e3, 2),
                       "tflops": round(flop / (chain_ms * 1e-3) / 1e12, 1),
                       "frac": round(flop / (chain_ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
                       "form": "pack, up-projection with GELU-tanh in its epilogue written packed, down-projection"}
    log(f"[bench] c4 GELU {gelu_ms*1e3:.1f} us; c4 chain {chain_ms*1e3:.1f} us "
        f"({out['c4_chain']['tflops']:.0f} TFLOP/s)")
    del a, wu, wd, y1, g, pa, ph, y2
    return out


def bench_configs(torch, b1, synth, steps, warmup):
    """The other config shapes, each from fp32 activations through
    bonsai_b1_linear_f32 (pack pass + GEMM; split along K where the shape
    asks for it): C1 (256 x 3072 -> 3072), C3 q/k/v and out-projection,
    C4 up- and down-projection, GELU-tanh between them, and the C4 chain in
    its fused form (GELU in the up-projection's epilogue, written as the
    down-projection's packed input); then the C5 38-block step."""
    out = {}
    for name, shp in [("c1_parity", (256, 3072, 3072)), ("c3_qkv", (4608, 3072, 9216)),
                      ("c3_out", (4608, 3072, 3072)), ("c4_up", (4608, 3072, 12288)),
                      ("c4_down", (4608, 12288, 3072))]:
        r = bench_gemm(torch, b1, synth, *shp, steps, warmup)
        out[name] = {"shape": list(shp), "us": round(r["ms"] * 1e3, 2), "tflops": round(r["tflops"], 1),
                     "frac": round(r["frac"], 4)}
        log(f"[bench] {name} {shp}: {r['ms']*1e3:.1f} us {r['tflops']:.1f} TFLOP/s ({100*r['frac']:.1f}% of peak)")
        del r
    out.update(bench_c4_mlp(torch, b1, synth))
    torch.cuda.empty_cache()
    c5 = bench_c5_block_chain(torch, b1, synth)
    out["c5_step"] = {x: (round(v, 4) if isinstance(v, float) else v) for x, v in c5.items()}
    log(f"[bench] c5 step (38 blocks): {c5['ms_per_step']:.2f} ms ({c5['gemm_tflops']:.0f} TFLOP/s of GEMM work, "
        f"{100*c5['frac']:.1f}% of peak); the 76 GEMMs alone {c5['ms_per_step_gemms_only']:.2f} ms")
    torch.cuda.empty_cache()
    kl = bench_klein_step(torch, b1, synth)
    out["klein_step"] = {x: round(v_, 4) if isinstance(v_, float) else v_ for x, v_ in kl.items()}
    log(f"[bench] Klein step (100 linears): {kl['ms_per_step']:.2f} ms ({kl['tflops']:.0f} TFLOP/s, "
        f"{100 * kl['frac']:.1f}% of peak); over producer-packed fp16 inputs {kl['ms_per_step_packed_inputs']:.2f} ms; "
        f"with FF-in and linear1 writing SwiGLU as the next packed input {kl['ms_per_step_swiglu_epilogues']:.2f} ms")
    torch.cuda.empty_cache()
    return out


def bench_exact(torch, b1, synth):
    """EXACT mode (b1_exact_kernel: fp32 VALU in the reference's scalar
    summation order, src/b1_0_kernel.h:240-287, bit-identical to it) at C1
    and at the headline shape, from fp32 activations; a few launches each
    after one warm-up (the headline takes milliseconds per launch)."""
    res = {}
    for name, (m, k, n), reps in (("c1", (256, 3072, 3072), 20), ("headline", HEADLINE, 3)):
        a = synth.device_activations(m, k, 31)
        w = synth.device_packed_weights(n, k, 32)
        y = torch.empty((m, n), device="cuda")
        ms, _ = time_launches(torch, lambda i: b1.linear(a, w, n, out=y, mode="exact"), reps, 1)
        tf = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        res[name] = {"shape": [m, k, n], "us": round(ms * 1e3, 1), "tflops": round(tf, 2),
                     "frac_fp32_valu": round(tf / PEAK_FP32_TFLOPS, 4), "launches": reps}
        log(f"[bench] EXACT mode {name} {(m, k, n)}: {ms * 1e3:.1f} us ({tf:.2f} TFLOP/s, "
            f"{100 * tf / PEAK_FP32_TFLOPS:.1f}% of the fp32 peak)")
        del a, w, y
    torch.cuda.empty_cache()
    return res


def bench_klein_step(torch, b1, synth):
    """The 100 B1_0 linears of one reference Flux.2-Klein step at 64x64
    latents (4096 image + 512 text tokens): 5 double-stream blocks (image and
    text q/k/v/out 3072 -> 3072, FF-in 3072 -> 18432, FF-out 9216 -> 3072)
    and 20 single-stream blocks (4608 x 3072 -> 27648, 12288 -> 3072), each
    with resident weights (690 MB), as one bonsai_b1_linear_batch call per
    step.  q, k and v of a stream read the same input; their weights are
    stored back to back (as bonsai_b1_weights_concat lays them out) and
    their outputs are adjacent column ranges, so the batch runs them as one
    GEMM over 9216 rows.  The same step with q/k/v writing separate outputs
    (three GEMMs sharing one packing) is timed beside it."""
    mi, mt, ms_ = 4096, 512, 4608
    d = []
    for blk in range(5):
        per = {}
        for st in ("img", "txt"):
            base = 1000 + 40 * blk + (20 if st == "txt" else 0)
            qkv = torch.cat([synth.device_packed_weights(3072, 3072, base + i).reshape(-1) for i in range(3)])
            per[st] = {"qkv": qkv,
                       "out": synth.device_packed_weights(3072, 3072, base + 3),
                       "ff_in": synth.device_packed_weights(18432, 3072, base + 4),
                       "ff_out": synth.device_packed_weights(3072, 9216, base + 5)}
        d.append(per)
    s = [(synth.device_packed_weights(27648, 3072, 2000 + i), synth.device_packed_weights(3072, 12288, 2100 + i))
         for i in range(20)]
    acts = {mm: {kk: synth.device_activations(mm, kk, 16 + kk) for kk in (3072, 9216, 12288)}
            for mm in (mi, mt, ms_)}
    outs = {mm: {nn: torch.empty((mm, nn), device="cuda") for nn in (3072, 9216, 18432, 27648)} for mm in (mi, mt, ms_)}
    ws = torch.empty(ms_ * 12288 * 2, dtype=torch.uint8, device="cuda")
    rs = 3072 // 32 * 6

    def step_ops(fuse_qkv):
        # graph order; attention and FF-in inputs are stand-ins of the right shapes
        ops = []
        attn = {mm: acts[mm][3072] for mm in (mi, mt)}
        for per in d:
            for st, mm in (("img", mi), ("txt", mt)):
                x = acts[mm][3072]
                for i in range(3):
                    wv = b1.device_weights(per[st]["qkv"][i * 3072 * rs:(i + 1) * 3072 * rs], 3072, 3072)
                    o = outs[mm][9216][:, i * 3072:(i + 1) * 3072] if fuse_qkv else outs[mm][3072]
                    ops.append((x, wv, o))
                ops.append((attn[mm], b1.device_weights(per[st]["out"], 3072, 3072), outs[mm][3072]))
                ops.append((x, b1.device_weights(per[st]["ff_in"], 3072, 18432), outs[mm][18432]))
                ops.append((acts[mm][9216], b1.device_weights(per[st]["ff_out"], 9216, 3072), outs[mm][3072]))
        for w1, w2 in s:
            ops.append((acts[ms_][3072], b1.device_weights(w1, 3072, 27648), outs[ms_][27648]))
            ops.append((acts[ms_][12288], b1.device_weights(w2, 12288, 3072), outs[ms_][3072]))
        assert len(ops) == 100
        return ops

    ops_f, ops_s = step_ops(True), step_ops(False)
    need = max(b1.linear_batch_workspace_bytes(ops_f), b1.linear_batch_workspace_bytes(ops_s))
    if need > ws.numel():
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    ms = graph_ms(torch, lambda: b1.linear_batch(ops_f, workspace=ws), reps=2)
    ms_sep = graph_ms(torch, lambda: b1.linear_batch(ops_s, workspace=ws), reps=2)
    # the same GEMMs over inputs already in the packed fp16 layout (as fused
    # producers write them), q/k/v as one GEMM: the step without pack passes
    packed = {}
    for mm in (mi, mt, ms_):
        for kk in (3072, 9216, 12288):
            packed[(mm, kk)] = b1.pack_act_f16(acts[mm][kk])
    gemms = []   # (packed input, weights, K, N, out)
    for per in d:
        for st, mm in (("img", mi), ("txt", mt)):
            gemms.append((packed[(mm, 3072)], per[st]["qkv"], 3072, 9216, outs[mm][9216]))
            gemms.append((packed[(mm, 3072)], per[st]["out"], 3072, 3072, outs[mm][3072]))
            gemms.append((packed[(mm, 3072)], per[st]["ff_in"], 3072, 18432, outs[mm][18432]))
            gemms.append((packed[(mm, 9216)], per[st]["ff_out"], 9216, 3072, outs[mm][3072]))
    for w1, w2 in s:
        gemms.append((packed[(ms_, 3072)], w1, 3072, 27648, outs[ms_][27648]))
        gemms.append((packed[(ms_, 12288)], w2, 12288, 3072, outs[ms_][3072]))
    assert len(gemms) == 80

    def step_packed():
        for pa, wt, kk, nn, o in gemms:
            b1.linear_packed_f16(pa, wt, kk, nn, o.shape[0], out=o)
    ms_packed = graph_ms(torch, step_packed, reps=2)

    # the same, with the MLP activations produced by the GEMMs that precede
    # them: FF-in and the single blocks' linear1 write SwiGLU of their MLP
    # columns straight into the packed input of FF-out / to_out (linear1's
    # q/k/v columns as fp32), as bonsai_b1_linear_packed_f16_to_packed does
    def step_packed_epilogue():
        for pa, wt, kk, nn, o in gemms:
            mm = o.shape[0]
            if nn == 18432:
                b1.linear_packed_f16_to_packed(pa, wt, kk, nn, mm, 0, "swiglu", packed_out=packed[(mm, 9216)])
            elif nn == 27648:
                b1.linear_packed_f16_to_packed(pa, wt, kk, nn, mm, 9216, "swiglu", out=outs[mm][9216],
                                               packed_out=packed[(mm, 12288)][3072 * 2:], ldp=12288)
            else:
                b1.linear_packed_f16(pa, wt, kk, nn, mm, out=o)
    ms_epi = graph_ms(torch, step_packed_epilogue, reps=2)
    flop = (5 * 2 * (mi + mt) * (4 * 3072 * 3072 + 3072 * 18432 + 9216 * 3072)
            + 20 * 2 * ms_ * (3072 * 27648 + 12288 * 3072))
    nbytes = sum(v.numel() for per in d for st in per.values() for v in st.values()) + \
        sum(a.numel() + b.numel() for a, b in s)
    return {"linears": 100, "ms_per_step": ms, "tflops": flop / (ms * 1e-3) / 1e12, "flop": flop,
            "frac": flop / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS,
            "ms_per_step_separate_qkv": ms_sep, "packed_weight_bytes": nbytes,
            "ms_per_step_packed_inputs": ms_packed, "tflops_packed_inputs": flop / (ms_packed * 1e-3) / 1e12,
            "ms_per_step_swiglu_epilogues": ms_epi, "tflops_swiglu_epilogues": flop / (ms_epi * 1e-3) / 1e12,
            "dispatch": "bonsai_b1_linear_batch, one call per step; q/k/v as one GEMM over concatenated weights"}


def bench_weights_load(torch, b1, blocks=38):
    """Weight residency for the C5 model's B1_0 tensors (38 blocks x
    [21504, 576] + [3072, 2880] packed bytes, 807 MB) from one .safetensors
    file in the page cache: bonsai_b1_safetensors_load (file mapped and
    parsed once, pinned staging) against one bonsai_b1_weights_upload per
    tensor straight from the mapping (pageable memory).  Each is timed from
    the call to the weights being resident; best of two."""
    import ctypes
    import mmap
    import shutil
    import tempfile
    import numpy as np
    from safetensors.numpy import save_file
    rng = np.random.default_rng(7)
    shapes = [(21504, 576), (3072, 2880)]
    tensors = {f"single_transformer_blocks.{i}.{nm}.weight": rng.integers(0, 256, shp, dtype=np.uint8)
               for i in range(blocks) for nm, shp in zip(("proj_mlp", "proj_out"), shapes)}
    nbytes = sum(t.nbytes for t in tensors.values())
    d = tempfile.mkdtemp(prefix="b1w")
    try:
        path = f"{d}/c5.safetensors"
        save_file(tensors, path)
        del tensors
        names = None
        r = {"tensors": 2 * blocks, "bytes": nbytes, "pinned_s": None, "pageable_s": None}
        with b1.SafetensorsFile(path) as f:
            names = f.names()
            spans = [f.find(nm) for nm in names]
            for _ in range(2):
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                ws = f.load(names)
                dt = time.perf_counter() - t0
                for w in ws:
                    b1.weights_free(w)
                r["pinned_s"] = dt if r["pinned_s"] is None else min(r["pinned_s"], dt)
        lib = b1.load()
        st = torch.cuda.current_stream()
        with open(path, "rb") as fh, mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ) as mm:
            base = np.frombuffer(mm, dtype=np.uint8)
            ptr = base.ctypes.data
            for _ in range(2):
                ws = []
                torch.cuda.synchronize()
                t0 = time.perf_counter()
                for (k, n, off, nb) in spans:
                    w = b1.capi.B1WeightsC()
                    assert lib.bonsai_b1_weights_upload(ptr + off, nb, k, n, ctypes.c_void_p(st.cuda_stream),
                                                        ctypes.byref(w)) == 0
                    ws.append(w)
                st.synchronize()
                dt = time.perf_counter() - t0
                for w in ws:
                    b1.weights_free(w)
                r["pageable_s"] = dt if r["pageable_s"] is None else min(r["pageable_s"], dt)
            del base
        r["pinned_GBps"] = nbytes / r["pinned_s"] / 1e9
        r["pageable_GBps"] = nbytes / r["pageable_s"] / 1e9
        return r
    finally:
        shutil.rmtree(d, ignore_errors=True)


def bench_gemv(torch, b1, synth, m, k, n, steps, warmup, packed_input=False, floor=False):
    """Small-M kernel, weight copies rotated past the MALL.  The launches are
    captured once into a HIP graph (one launch per weight copy) and the graph
    is replayed, so the GPU runs the kernels back to back with no host in the
    loop; the per-launch time is the event time over the replays / launches.
    packed_input: the activations arrive in the packed fp16 layout (from a
    producer) and bonsai_b1_linear_packed_f16 runs the same kernel without
    the conversion.  floor: also the plain read of the same copies
    (read_floor)."""
    nbytes = n * (k // 32) * 6
    copies = max(2, (2 * MALL_BYTES) // nbytes + 1)      # rotate > 2x the MALL
    ws = [synth.device_packed_weights(n, k, 100 + c) for c in range(copies)]
    a = synth.device_activations(m, k, 3)
    pa = b1.pack_act_f16(a) if packed_input else None
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")

    def call(c):
        if packed_input:
            b1.linear_packed_f16(pa, ws[c], k, n, m, out=y)
        else:
            b1.linear(a, ws[c], n, out=y, mode="gemv")
    call(0)                                              # load the code object
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for c in range(copies):
            call(c)
    reps = max(1, steps // copies)
    ms, wall = time_launches(torch, lambda i: graph.replay(), reps, max(1, warmup // copies))
    ms /= copies
    eager_ms, _ = time_launches(torch, lambda i: call(i % copies), steps, warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"shape": [m, k, n], "ms": ms, "us": ms * 1e3, "gbs": gbs, "frac": gbs / PEAK_HBM_GBS,
           "packed_bytes": nbytes, "weight_copies": copies, "launches": reps * copies,
           "eager_us": eager_ms * 1e3, "wall_s": wall}
    if floor:
        res["read_floor"] = read_floor(torch, ws, nbytes, steps, warmup)
    return res


MOD_GROUP = (1, 3072, [18432, 18432, 9216, 6144])   # a step's modulation projections over vec_silu


def bench_gemv_group(torch, b1, synth, m, k, ns, steps, warmup):
    """Consecutive small-M linears on one input (a diffusion step's
    modulation projections): one bonsai_b1_linear_batch call, which runs them
    as one launch (over the fp32 input itself at m <= 8, else over one
    packing of it), against the same linears as separate calls.  Weight sets rotated past the MALL, launches captured in
    a HIP graph as in bench_gemv."""
    nbytes = sum(n * (k // 32) * 6 for n in ns)
    copies = max(2, (2 * MALL_BYTES) // nbytes + 1)
    wsets = [[synth.device_packed_weights(n, k, 500 + 10 * c + i) for i, n in enumerate(ns)] for c in range(copies)]
    a = synth.device_activations(m, k, 5)
    outs = [torch.empty((m, n), dtype=torch.float32, device="cuda") for n in ns]
    views = [[b1.device_weights(w, k, n) for w, n in zip(ws, ns)] for ws in wsets]
    ops = [[(a, v, o) for v, o in zip(vs, outs)] for vs in views]
    wsp = torch.empty(max(16, b1.linear_batch_workspace_bytes(ops[0])), dtype=torch.uint8, device="cuda")

    def grouped(c):
        b1.linear_batch(ops[c], workspace=wsp)

    def separate(c):
        for w, n, o in zip(wsets[c], ns, outs):
            b1.linear(a, w, n, out=o)
    res = {}
    for name, fn in (("grouped", grouped), ("separate", separate)):
        fn(0)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for c in range(copies):
                fn(c)
        reps = max(1, steps // copies)
        ms, _ = time_launches(torch, lambda i: graph.replay(), reps, max(1, warmup // copies))
        res[name] = ms / copies
    ref = [o.clone() for o in outs]
    grouped(copies - 1)
    torch.cuda.synchronize()
    same = all(torch.equal(o, r) for o, r in zip(outs, ref))
    del wsets, views, ops
    flat = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(copies)]
    floor = read_floor(torch, flat, nbytes, steps, warmup)
    del flat
    return {"shape": [m, k, ns], "grouped_us": res["grouped"] * 1e3, "separate_us": res["separate"] * 1e3,
            "grouped_GBps": nbytes / (res["grouped"] * 1e-3) / 1e9,
            "separate_GBps": nbytes / (res["separate"] * 1e-3) / 1e9, "packed_bytes": nbytes,
            "weight_sets": copies, "grouped_equals_separate": same, "read_floor": floor}


def bench_dense_reference(torch, m, k, n, steps=1000, warmup=3000):
    """The vendor library's dense GEMM at the headline shape on the same
    GPU, for context: torch.mm over fp16 operands (hipBLASLt), fp32 output
    like the B1_0 op's, weights [N, K] used transposed as a linear layer
    does.  No B1_0 decode is involved."""
    a = torch.randn(m, k, device="cuda", dtype=torch.float16)
    wt = torch.randn(n, k, device="cuda", dtype=torch.float16).t()
    try:
        out = torch.empty((m, n), device="cuda", dtype=torch.float32)
        torch.mm(a, wt, out_dtype=torch.float32, out=out)
        fn, out_dtype = (lambda: torch.mm(a, wt, out_dtype=torch.float32, out=out)), "fp32"
    except (TypeError, RuntimeError):
        out = torch.empty((m, n), device="cuda", dtype=torch.float16)
        fn, out_dtype = (lambda: torch.mm(a, wt, out=out)), "fp16"
    ms, _ = time_launches(torch, lambda i: fn(), steps, warmup)
    return {"library": "hipBLASLt via torch.mm", "operands": "fp16", "out": out_dtype, "us": ms * 1e3,
            "tflops": 2.0 * m * n * k / (ms * 1e-3) / 1e12}


def bench_copy(torch, nbytes, steps, warmup):
    """Plain device copy of known size: calibrates the FETCH_SIZE/WRITE_SIZE
    counters (bytes moved = nbytes read + nbytes written per launch)."""
    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").uniform_()
    dst = torch.empty_like(src)
    ms, _ = time_launches(torch, lambda i: dst.copy_(src), steps, warmup)
    return {"bytes": nbytes, "ms": ms, "gbs": 2 * nbytes / (ms * 1e-3) / 1e9}


def observed_sclk_mhz():
    """The shader clock now, in MHz: the current level of the amdgpu sysfs
    DPM table (the line marked '*'), else the mean of amd-smi's per-XCD
    current clocks, else rocm-smi's; None if none answers."""
    import glob
    import re
    import subprocess
    for f in sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk")):
        try:
            for line in open(f):
                if line.rstrip().endswith("*"):
                    m = re.search(r"(\d+)\s*mhz", line, re.I)
                    if m:
                        return int(m.group(1))
        except OSError:
            pass
    try:
        out = subprocess.run(["amd-smi", "metric", "-c", "-g", "0", "--json"], capture_output=True, text=True,
                             timeout=20).stdout
        data = json.loads(out)
        gpu = data["gpu_data"][0] if isinstance(data, dict) else data[0]
        clks = [v["clk"]["value"] for k, v in gpu["clock"].items() if k.startswith("gfx")]
        if clks:
            return int(round(sum(clks) / len(clks)))
    except Exception:
        pass
    try:
        out = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True, timeout=20).stdout
        m = re.search(r"sclk clock level:.*?\((\d+)Mhz\)", out)
        return int(m.group(1)) if m else None
    except Exception:
        return None


def settle_clock(torch, fn, seconds):
    """Runs fn back to back for `seconds` of wall time, so that the shader
    clock has ramped and settled under sustained MFMA load before anything
    is timed, and reads the clock once while the GPU is still busy (the
    reading runs in a thread; the launches go on until it has returned).
    Returns (seconds spent, clock in MHz or None)."""
    import threading
    sclk = []
    th = threading.Thread(target=lambda: sclk.append(observed_sclk_mhz()), daemon=True)
    t0 = time.perf_counter()
    started = False
    i = 0
    while True:
        for _ in range(8):
            fn(i)
            i += 1
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
        if not started and el >= 0.5 * seconds:
            th.start()
            started = True
        if el >= seconds and started and not th.is_alive():
            break
    th.join()
    return time.perf_counter() - t0, (sclk[0] if sclk else None)


def cpu_time(fn, reps):
    """Median wall time of fn over reps runs, after one warm-up run."""
    import numpy as np
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts))


def cpu_baselines(a_dev, w_dev, n, threads_share):
    """The oracle's AVX2 restatement of src/b1_0_kernel.h:79-239 (ggml row
    split over nth threads, :75-77) on this host, on the same device inputs
    the GPU legs timed (copied to host): the headline GEMM on all 4096 rows
    at the host's thread share, on its first 1024 rows at nth = 4 (the
    reference's --threads default, src/diffuser.cpp:63), and the M=8
    small-M shape (K=3072, N=18432) at both thread counts, median of 3."""
    import numpy as np
    from bonsai_b1 import synth
    from oracle import b1_oracle as o
    k = a_dev.shape[1]
    act = a_dev.cpu().numpy()
    raw = w_dev.cpu().numpy().reshape(n, -1)

    def run(a, r, nn, th):
        return lambda: o.linear(a, r, nn, variant="avx2", nth=th, nthreads=th)
    res = {}
    for th, rows in ((threads_share, act.shape[0]), (4, 1024)):
        dt = cpu_time(run(act[:rows], raw, n, th), 3)
        res[th] = {"tflops": 2.0 * rows * n * k / dt / 1e12, "s": dt, "rows": rows}
    gm, gk, gn = GEMV
    ga = synth.activations(gm, gk, 3)
    graw = synth.packed_weights(gn, gk, 4)
    nbytes = gn * (gk // 32) * 6
    gemv = {}
    for th in (threads_share, 4):
        # a call takes milliseconds, most of it thread start-up and the
        # first touch of 10.6 MB: the median of many is the stable figure
        dt = cpu_time(run(ga, graw, gn, th), 25)
        gemv[th] = {"us": dt * 1e6, "GBps_packed": nbytes / dt / 1e9, "reps": 25}
    return res, gemv


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo, else lscpu), or None."""
    try:
        for line in open("/proc/cpuinfo"):
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    try:
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.lower().startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    # the shader clock ramps for about a second under sustained MFMA load
    # before it settles; nothing is timed before this much wall time of it
    ap.add_argument("--settle-s", type=float, default=2.0)
    ap.add_argument("--all", action="store_true", help="also time the secondary legs (stderr and JSON)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-configs", action="store_true", help="skip the C1/C3/C4/C5 config legs")
    ap.add_argument("--only", choices=["gemm", "gemv", "copy", "c5chain", "tiles16", "c4", "exact"], default=None,
                    help="run one leg only (profiler runs); prints that leg's numbers")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the B1_0 linear is built and timed on a single "
              "MI355X; sharding across GPUs is designed but not built.", file=sys.stderr)
        sys.exit(2)

    import torch
    import bonsai_b1 as b1
    from bonsai_b1 import synth
    b1.load()
    torch.cuda.init()

    m, k, n = HEADLINE
    if args.only == "copy":
        c = bench_copy(torch, 256 << 20, args.steps, args.warmup)
        print(json.dumps({"copy": c}), flush=True)
        return
    if args.only == "tiles16":
        a = synth.device_activations(4608, 3072, 1)
        w = synth.device_packed_weights(3072, 3072, 2)
        settle_s, sclk = settle_clock(torch, lambda i: b1.linear(a, w, 3072), args.settle_s)
        del a, w
        t16 = bench_tiles16(torch, b1, synth, args.steps, args.warmup)
        print(json.dumps({"tiles16": t16, "sclk_mhz": sclk}), flush=True)
        return
    if args.only == "exact":
        print(json.dumps({"exact": bench_exact(torch, b1, synth)}), flush=True)
        return
    if args.only == "c4":
        c4 = bench_c4_mlp(torch, b1, synth, reps=max(4, args.steps // 10))
        print(json.dumps({"c4": c4}), flush=True)
        return
    if args.only == "c5chain":
        ch = bench_c5_block_chain(torch, b1, synth, producer_form=True)
        print(json.dumps({"c5_block_chain": ch}), flush=True)
        return
    if args.only == "gemv":
        gm, gk, gn = GEMV
        v = bench_gemv(torch, b1, synth, gm, gk, gn, max(args.steps, 200), min(args.warmup, 400), floor=True)
        vp = bench_gemv(torch, b1, synth, gm, gk, gn, max(args.steps, 200), min(args.warmup, 400),
                        packed_input=True)
        v1 = bench_gemv(torch, b1, synth, 1, gk, gn, max(args.steps, 200), min(args.warmup, 400))
        vg = bench_gemv_group(torch, b1, synth, *MOD_GROUP, max(args.steps, 200), min(args.warmup, 400))
        print(json.dumps({"gemv": {x: v[x] for x in v}, "gemv_packed": {x: vp[x] for x in vp},
                          "gemv_m1": {x: v1[x] for x in v1}, "modulation_group": vg}), flush=True)
        return
    a = synth.device_activations(m, k, 1)
    w = synth.device_packed_weights(n, k, 2)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    settle_s, sclk = settle_clock(torch, lambda i: b1.linear(a, w, n, out=y), args.settle_s)
    log(f"[bench] clock settled over {settle_s:.2f} s of the step (sclk under load: {sclk} MHz)")
    log(f"[bench] GEMM M={m} K={k} N={n} steps={args.steps} warmup={args.warmup}")
    g = bench_gemm(torch, b1, synth, m, k, n, args.steps, args.warmup, inputs=(a, w))
    log(f"[bench] GEMM {g['ms']*1e3:.1f} us  {g['tflops']:.1f} TFLOP/s  {100*g['frac']:.1f}% of fp16 MFMA peak")
    # the kernels alone: at least 100 launches each for a stable event average
    kern_ms, pack_ms = bench_step_kernels(torch, b1, a, w, n, max(args.steps, 100), max(args.warmup, 10))
    kern_tflops = 2.0 * m * n * k / (kern_ms * 1e-3) / 1e12
    pack_gbs = m * k * 6 / (pack_ms * 1e-3) / 1e9
    log(f"[bench] GEMM kernel alone {kern_ms*1e3:.1f} us  {kern_tflops:.1f} TFLOP/s  "
        f"{100*kern_tflops/PEAK_FP16_TFLOPS:.1f}% of peak; pack pass alone {pack_ms*1e3:.1f} us "
        f"({pack_gbs:.0f} GB/s)")
    if args.only == "gemm":
        print(json.dumps({"gemm": {x: g[x] for x in g if x != "inputs"}, "kernel_ms": kern_ms,
                          "pack_ms": pack_ms, "sclk_mhz": sclk}), flush=True)
        return
    dense = bench_dense_reference(torch, m, k, n, steps=max(args.steps, 100), warmup=max(args.warmup, 50))
    log(f"[bench] dense fp16 GEMM, same shape ({dense['library']}, {dense['out']} out): {dense['us']:.1f} us "
        f"{dense['tflops']:.1f} TFLOP/s; B1_0 kernel / dense = {kern_ms * 1e3 / dense['us']:.3f}")

    gm, gk, gn = GEMV
    log(f"[bench] GEMV M={gm} K={gk} N={gn}")
    v = bench_gemv(torch, b1, synth, gm, gk, gn, max(args.steps, 200), min(args.warmup, 400), floor=True)
    log(f"[bench] GEMV {v['us']:.2f} us/launch (graph)  {v['gbs']:.0f} GB/s packed  "
        f"{100*v['frac']:.1f}% of HBM peak; eager {v['eager_us']:.2f} us/call; a plain read of the same "
        f"bytes {v['read_floor']['us']:.2f} us/launch ({100 * v['read_floor']['frac_hbm']:.1f}% of HBM peak)")
    v1 = bench_gemv(torch, b1, synth, 1, gk, gn, max(args.steps, 200), min(args.warmup, 400))
    log(f"[bench] GEMV M=1 {v1['us']:.2f} us/call  {v1['gbs']:.0f} GB/s packed")
    vp = bench_gemv(torch, b1, synth, gm, gk, gn, max(args.steps, 200), min(args.warmup, 400), packed_input=True)
    log(f"[bench] GEMV M={gm} over packed fp16 activations {vp['us']:.2f} us/launch  {vp['gbs']:.0f} GB/s "
        f"({100 * vp['frac']:.1f}% of HBM peak)")
    vg = bench_gemv_group(torch, b1, synth, *MOD_GROUP, max(args.steps, 200), min(args.warmup, 400))
    log(f"[bench] modulation projections M={MOD_GROUP[0]} K={MOD_GROUP[1]} N={MOD_GROUP[2]}: one batch call "
        f"{vg['grouped_us']:.2f} us ({vg['grouped_GBps']:.0f} GB/s), separate calls {vg['separate_us']:.2f} us "
        f"({vg['separate_GBps']:.0f} GB/s); equal {vg['grouped_equals_separate']}; a plain read of the same "
        f"bytes {vg['read_floor']['us']:.2f} us/launch")

    configs = {}
    if not args.no_configs:
        configs = bench_configs(torch, b1, synth, max(args.steps // 4, 20), max(args.warmup, 10))
    if args.all:
        mlp = bench_mlp(torch, b1, synth)
        configs["c4_mlp_forms"] = {x: round(v_, 4) for x, v_ in mlp.items()}
        log(f"[bench] c4 MLP forms: chain {mlp['chain']*1e3:.1f} us, GELU fused into the pack "
            f"{mlp['chain_fused_gelu']*1e3:.1f} us, GELU in the up-projection's epilogue "
            f"{mlp['chain_epilogue_gelu']*1e3:.1f} us")
        ff = bench_ff_epilogues(torch, b1, synth)
        configs["ff_epilogues"] = {x: round(v_, 4) for x, v_ in ff.items()}
        log(f"[bench] double-block FF (4096 x 3072 -> 2x9216, SwiGLU, -> 3072, gate-residual): separate "
            f"passes {ff['separate']*1e3:.1f} us, fused epilogues {ff['fused']*1e3:.1f} us "
            f"({ff['fused_tflops']:.0f} TFLOP/s); SwiGLU epilogue writing FF-out's packed input "
            f"{ff['fused_packed_out']*1e3:.1f} us ({ff['fused_packed_out_tflops']:.0f} TFLOP/s)")
        nm = bench_norm_mod(torch, b1, synth)
        configs["norm_mod"] = {x: round(v_, 4) for x, v_ in nm.items()}
        log(f"[bench] LayerNorm+modulation 4096x3072 -> packed fp16: {nm['fused_pack']*1e3:.1f} us "
            f"({nm['fused_GBps']:.0f} GB/s); fp32 then pack {nm['fp32_then_pack']*1e3:.1f} us")
        torch.cuda.empty_cache()
        c5 = bench_single_stream_step(torch, b1, synth)
        configs["c5_step_fp32_inputs"] = {x: round(v_, 4) if isinstance(v_, float) else v_ for x, v_ in c5.items()}
        log(f"[bench] c5 38 blocks of (linear1, linear2) from fp32 activations: {c5['ms_per_step']:.2f} ms "
            f"({c5['tflops']:.0f} TFLOP/s)")
        torch.cuda.empty_cache()
        wl = bench_weights_load(torch, b1)
        configs["weights_load"] = {x: round(v_, 4) if isinstance(v_, float) else v_ for x, v_ in wl.items()}
        log(f"[bench] weight residency, C5 model ({wl['tensors']} tensors, {wl['bytes'] / 1e6:.0f} MB) from "
            f".safetensors: pinned pipeline {wl['pinned_s'] * 1e3:.0f} ms ({wl['pinned_GBps']:.1f} GB/s), "
            f"per-tensor upload from the mapping {wl['pageable_s'] * 1e3:.0f} ms ({wl['pageable_GBps']:.1f} GB/s)")
        torch.cuda.empty_cache()
    exact = None if args.no_configs else bench_exact(torch, b1, synth)

    cpu = None
    if not args.no_cpu:
        share = min(16, len(os.sched_getaffinity(0)))
        log(f"[bench] CPU baseline: oracle AVX2, {share} and 4 threads")
        res, gemv_cpu = cpu_baselines(a, w, n, share)
        top = res[share]
        cpu = {"value": round(top["tflops"], 5), "unit": "TFLOP/s", "cores": share, "kind": "port",
               "host_cpus": os.cpu_count(), "cpu_model": cpu_model(),
               "sample": f"M={top['rows']} of {m} rows, K={k}, N={n}; AVX2 restatement of "
                         f"src/b1_0_kernel.h:79-239, gcc -O3 -mavx2 -mfma -mf16c -ffp-contract=off, "
                         f"ggml row split nth={share}; median of 3 ({top['s']:.2f} s)",
               "nth4": {"value": round(res[4]["tflops"], 5), "unit": "TFLOP/s",
                        "sample": f"M={res[4]['rows']} rows, nth=4 (src/diffuser.cpp:63 default); "
                                  f"median of 3 ({res[4]['s']:.2f} s)"},
               "gemv_m8": {f"nth{th}": {"us": round(r_["us"], 1), "GBps_packed": round(r_["GBps_packed"], 2)}
                           for th, r_ in gemv_cpu.items()}}
        log(f"[bench] CPU {top['tflops']*1e3:.1f} GFLOP/s at {share} threads, {res[4]['tflops']*1e3:.1f} at 4; "
            f"GEMV M=8 {gemv_cpu[share]['us']:.0f} us at {share} threads")

    flop = 2.0 * m * n * k
    line = {
        "metric": "B1_0 GEMM TFLOP/s & % roofline at M4096 K3072 N12288; GEMV GB/s % HBM peak",
        "value": round(g["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(g["ms"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16-mfma/fp32-acc",
        "data": "synthetic (N(0,1) fp32 activations, random B1_0 packed weights)",
        "config": {"workload": "b1_0_gemm", "M": m, "K": k, "N": n, "mode": "fast",
                   "parallelism": "single-gpu"},
        "settle_s": round(settle_s, 3),
        "sclk_mhz_under_load": sclk,
        "roofline": {"bound": "mfma", "achieved": round(kern_tflops, 2), "peak": PEAK_FP16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(kern_tflops / PEAK_FP16_TFLOPS, 4),
                     "traffic": committed_traffic(TRAFFIC_PROFILE),
                     "kernel": "b1_gemm_kernel<128,512,64,3,0>", "kernel_us": round(kern_ms * 1e3, 2),
                     "algorithmic_flop": flop, "traffic_source": f"profiles/{TRAFFIC_PROFILE}.md",
                     "pack_pass": {"kernel": "b1_pack_rows_kernel", "us": round(pack_ms * 1e3, 2),
                                   "GBps": round(pack_gbs, 1), "frac_hbm": round(pack_gbs / PEAK_HBM_GBS, 4),
                                   "algorithmic_bytes": m * k * 6},
                     "note": "value/ms_per_step: whole op from fp32 activations (pack pass + GEMM); "
                             "achieved: GEMM kernel alone; pack_pass: the other kernel of the step, alone"},
        "dense_reference": {x: (round(y_, 2) if isinstance(y_, float) else y_) for x, y_ in dense.items()},
        "gemv": {"M": gm, "K": gk, "N": gn, "us_per_call": round(v["us"], 3),
                 "GBps_packed": round(v["gbs"], 1), "frac_hbm": round(v["frac"], 4),
                 "packed_bytes": v["packed_bytes"], "weight_copies": v["weight_copies"],
                 "timing": "hip graph of back-to-back launches, one per weight copy",
                 "eager_us_per_call": round(v["eager_us"], 3),
                 "M1_us_per_call": round(v1["us"], 3), "M1_GBps_packed": round(v1["gbs"], 1),
                 "packed_input_us_per_call": round(vp["us"], 3), "packed_input_GBps": round(vp["gbs"], 1),
                 "packed_input_frac_hbm": round(vp["frac"], 4),
                 "read_floor": {"us_per_call": round(v["read_floor"]["us"], 3),
                                "GBps": round(v["read_floor"]["GBps"], 1),
                                "frac_hbm": round(v["read_floor"]["frac_hbm"], 4),
                                "grid": v["read_floor"]["grid"],
                                "note": "a kernel that only reads the same packed bytes, same graph replay over the "
                                        "same copies: what one launch of this size can reach on this GPU"},
                 "modulation_group": {"M": MOD_GROUP[0], "K": MOD_GROUP[1], "N": MOD_GROUP[2],
                                      "batch_call_us": round(vg["grouped_us"], 3),
                                      "batch_call_GBps": round(vg["grouped_GBps"], 1),
                                      "separate_calls_us": round(vg["separate_us"], 3),
                                      "separate_calls_GBps": round(vg["separate_GBps"], 1),
                                      "equal": vg["grouped_equals_separate"],
                                      "read_floor_us": round(vg["read_floor"]["us"], 3),
                                      "read_floor_GBps": round(vg["read_floor"]["GBps"], 1)}},
        "cpu_baseline": cpu,
    }
    if exact:
        line["exact"] = exact
    if configs:
        line["configs"] = configs
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
