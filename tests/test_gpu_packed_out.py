"""GPU checks of the GEMM epilogue that writes the next linear's packed fp16
activations (bonsai_b1_linear_packed_f16_to_packed).

Bar (bit for bit): the fp32 columns equal the plain GEMM's output (the same
tile kernel, the same K order), and the packed columns equal the packing
the separate producers write from that output -- bonsai_b1_pack_act_f16_ld,
bonsai_b1_gelu_tanh_pack_f16_ld or bonsai_b1_swiglu_pack_f16_ld -- which
the producer tests pin against the oracle's layout.  Bytes outside the
written column range keep their sentinel.  The shapes cover ragged row
counts, a few rows, split points inside a 512-column tile, the C5 single
block's linear1 (q/k/v fp32, GELU(MLP) into linear2's input at column
3072) and the reference single block's linear1 (SwiGLU MLP,
src/diffuser_graph.cpp:482-534).
"""
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
def b1(torch):
    import bonsai_b1
    bonsai_b1.load()
    return bonsai_b1


def produce(b1, y, act, packed, ldp):
    """The separate producer of the packed columns from the fp32 output."""
    if act == "none":
        b1.pack_act_f16(y, packed=packed, ldp=ldp)
    elif act == "gelu_tanh":
        b1.gelu_tanh_pack_f16(y, packed=packed, ldp=ldp)
    else:
        b1.swiglu_pack_f16(y, packed=packed, ldp=ldp)


# (m, k, n, split, act, column offset of the packed range, ldp or None)
CASES = [
    (300, 768, 1536, 512, "gelu_tanh", 0, None),
    (300, 768, 1536, 0, "none", 0, None),
    (300, 768, 1536, 96, "gelu_tanh", 0, None),      # split inside a tile
    (300, 768, 1536, 1536, "none", 0, None),         # fp32 columns only
    (5, 384, 1024, 0, "gelu_tanh", 0, None),         # a few rows
    (300, 768, 1536, 512, "swiglu", 0, None),
    (256, 768, 2048, 192, "swiglu", 64, 1216),       # SwiGLU split inside a tile, into a column range
    (600, 3072, 21504, 9216, "gelu_tanh", 3072, 15360),  # C5 linear1 -> linear2's input
    (600, 3072, 27648, 9216, "swiglu", 3072, 12288),     # reference single block linear1 -> to_out's input
    # 16x16 tile kernels (GELU and none; the plain reference runs the same
    # kernel): 144 x 384 and 128 x 384 tiles, every column packed; split
    # inside a wave (a block's halves in two waves: 2-byte half stores);
    # a wave with one fp32 tile and one packed block (fewer stores than a
    # full tile's: the next tile waits for everything); several tiles a
    # work-group
    (288, 384, 768, 0, "gelu_tanh", 0, None),
    (288, 384, 768, 416, "gelu_tanh", 0, None),
    (288, 384, 768, 448, "none", 32, 400),
    (512, 384, 768, 0, "gelu_tanh", 0, None),
    (512, 384, 768, 160, "gelu_tanh", 96, 800),
    (2048, 384, 9216, 4096, "gelu_tanh", 0, None),
    (4608, 384, 9216, 3072, "gelu_tanh", 0, None),
    # no activation, tiles wholly past the split point (the owner layout)
    (512, 384, 768, 0, "none", 0, None),
    (288, 384, 1152, 384, "none", 0, None),
    # SwiGLU on 16x16 tiles (split on a 384-column tile boundary): every
    # wave's 24 gates paired with their values, written as fp16 halves
    (512, 384, 768, 0, "swiglu", 0, None),
    (288, 384, 1152, 384, "swiglu", 0, None),
    (512, 384, 1536, 768, "swiglu", 32, 432),
    (4608, 384, 18432, 9216, "swiglu", 0, None),
    # packed rows of 2^22 + 32 fp16 elements, past the range of a buffer
    # resource over a tile's rows: the element-by-element stores
    (288, 384, 768, 0, "gelu_tanh", 0, 2**22 + 32),
    (512, 384, 1536, 0, "swiglu", 0, 2**22 + 32),
]


def _sweep(count=10, seed=2024):
    """Seeded extra cases: row counts around tile edges, widths and split
    points on 32- (64- for SwiGLU) column boundaries, column offsets and
    padded row strides."""
    import random
    rng = random.Random(seed)
    cases = []
    for _ in range(count):
        act = rng.choice(["none", "gelu_tanh", "swiglu"])
        q = 64 if act == "swiglu" else 32
        m = rng.choice([1, 17, 127, 128, 129, 255, 383, 640])
        k = rng.choice([384, 768, 1152])
        n = q * rng.randint(2, 48)
        split = q * rng.randint(0, n // q)
        cols = (n - split) // 2 if act == "swiglu" else n - split
        col0 = 32 * rng.randint(0, 3)
        ldp = None if col0 == 0 and rng.random() < 0.5 else col0 + cols + 8 * rng.randint(0, 8)
        if ldp is None:
            col0 = 0
        cases.append((m, k, n, split, act, col0, ldp))
    return cases


@pytest.mark.parametrize("m,k,n,split,act,col0,ldp", CASES + _sweep())
def test_packed_output_equals_linear_then_producer(torch, b1, m, k, n, split, act, col0, ldp):
    from bonsai_b1 import synth
    say(f"packed-output linear m={m} k={k} n={n} split={split} act={act} col0={col0} ldp={ldp}")
    a = synth.device_activations(m, k, 81)
    w = synth.device_packed_weights(n, k, 82)
    p = b1.pack_act_f16(a)
    y = b1.linear_packed_f16_epi(p, w, k, n, m, "none")
    cols = (n - split) // 2 if act == "swiglu" else n - split
    ld = ldp if ldp is not None else cols
    nbytes = max(((m - 1) * ld + col0 + cols) * 2, 16)
    got = torch.full((nbytes,), 0xA5, dtype=torch.uint8, device="cuda")
    want = got.clone()
    out = torch.full((m, split + 8), float("nan"), device="cuda") if split else None
    out_v = out[:, :split] if split else None
    b1.linear_packed_f16_to_packed(p, w, k, n, m, split, act, out=out_v, packed_out=got[col0 * 2:],
                                   ldp=ldp)
    if cols:
        produce(b1, y[:, split:], act, want[col0 * 2:], ld if ldp is not None else None)
    torch.cuda.synchronize()
    if split:
        assert torch.equal(out[:, :split], y[:, :split])
        assert torch.isnan(out[:, split:]).all()     # columns past split untouched
    assert torch.equal(got, want)


@pytest.mark.parametrize("act", ["gelu_tanh", "swiglu"])
def test_packed_output_counts_nonfinite_outputs(torch, b1, act):
    """The counter counts y, fp32 and packed columns alike: the plain GEMM's count."""
    from bonsai_b1 import synth
    m, k, n, split = 200, 768, 1536, 512
    say(f"packed-output non-finite count act={act}")
    a = synth.device_activations(m, k, 83)
    a[7, 100] = 1e6                                   # fp16 inf after packing
    a[150, 5] = -1e6
    w = synth.device_packed_weights(n, k, 84)
    p = b1.pack_act_f16(a)
    c_plain = torch.zeros(1, dtype=torch.int32, device="cuda")
    c_fused = torch.zeros(1, dtype=torch.int32, device="cuda")
    b1.linear_packed_f16_epi(p, w, k, n, m, "none", nonfinite=c_plain)
    b1.linear_packed_f16_to_packed(p, w, k, n, m, split, act, nonfinite=c_fused)
    torch.cuda.synchronize()
    assert int(c_plain.item()) == 2 * n
    assert int(c_fused.item()) == int(c_plain.item())


def test_packed_output_repeats_bit_identically(torch, b1):
    """Two launches over the same inputs, the second with fewer rows, agree."""
    from bonsai_b1 import synth
    k, n, split = 3072, 21504, 9216
    say("packed-output repeat")
    a = synth.device_activations(520, k, 85)
    w = synth.device_packed_weights(n, k, 86)
    p = b1.pack_act_f16(a)
    o1, q1 = b1.linear_packed_f16_to_packed(p, w, k, n, 520, split, "gelu_tanh")
    o2, q2 = b1.linear_packed_f16_to_packed(p, w, k, n, 260, split, "gelu_tanh")
    torch.cuda.synchronize()
    assert torch.equal(o1[:260], o2)
    assert torch.equal(q1[:q2.numel()], q2)


def test_packed_output_in_captured_graph(torch, b1):
    """The entry allocates nothing, so it can be captured: three replays,
    each after eager work on the same buffers, equal the eager result."""
    from bonsai_b1 import synth
    m, k, n, split = 384, 768, 2048, 512
    say("packed-output graph capture")
    a = synth.device_activations(m, k, 87)
    w = synth.device_packed_weights(n, k, 88)
    p = b1.pack_act_f16(a)
    out = torch.empty((m, split), device="cuda")
    pk = torch.empty(m * (n - split) * 2, dtype=torch.uint8, device="cuda")
    b1.linear_packed_f16_to_packed(p, w, k, n, m, split, "gelu_tanh", out=out, packed_out=pk)
    torch.cuda.synchronize()
    want_o, want_p = out.clone(), pk.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        b1.linear_packed_f16_to_packed(p, w, k, n, m, split, "gelu_tanh", out=out, packed_out=pk)
    for rep in range(3):
        out.fill_(float("nan"))
        pk.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want_o), f"replay {rep}"
        assert torch.equal(pk, want_p), f"replay {rep}"


@pytest.mark.parametrize("m,mode,act", [(300, "auto", "gelu_tanh"), (300, "auto", "swiglu"),
                                        (300, "exact", "gelu_tanh"), (96, "exact", "swiglu"),
                                        (5, "auto", "swiglu"), (5, "auto", "none")])
def test_packed_epilogue_of_fp32_entry(torch, b1, m, mode, act):
    """bonsai_b1_linear_epi_f32 with the packed-output epilogue: the fused
    FAST path equals pack + bonsai_b1_linear_packed_f16_to_packed; EXACT
    mode and the small-batch kernel (separate passes over the linear's
    output) equal that mode's own linear followed by the producers."""
    from bonsai_b1 import synth
    k, n, split, col0, ldp = 768, 2048, 512, 64, 1600
    say(f"packed epilogue, fp32 entry m={m} mode={mode} act={act}")
    a = synth.device_activations(m, k, 91)
    w = synth.device_packed_weights(n, k, 92)
    cols = (n - split) // 2 if act == "swiglu" else n - split
    nbytes = ((m - 1) * ldp + col0 + cols) * 2
    got = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device="cuda")
    want = got.clone()
    out = torch.full((m, split), float("nan"), device="cuda")
    e = b1.packed_epilogue(split, act, got[col0 * 2:], ldp)
    b1.linear_epi(a, w, n, e, out=out, mode=mode)
    if mode == "auto" and m > 16:
        o2, _ = b1.linear_packed_f16_to_packed(b1.pack_act_f16(a), w, k, n, m, split, act,
                                               packed_out=want[col0 * 2:], ldp=ldp)
        y_head = o2
    else:
        y = b1.linear(a, w, n, mode=mode)
        y_head = y[:, :split]
        produce(b1, y[:, split:], act, want[col0 * 2:], ldp)
    torch.cuda.synchronize()
    assert torch.equal(out, y_head)
    assert torch.equal(got, want)


def test_packed_epilogue_in_batch(torch, b1):
    """A batch with packed-output ops (q/k/v + SwiGLU MLP of a single block,
    a double block's FF-in) beside plain ops equals the ops one by one."""
    from bonsai_b1 import synth
    m, k = 320, 768
    say("packed epilogue in a batch")
    a = synth.device_activations(m, k, 93)
    a2 = synth.device_activations(m, k, 94)
    w1 = synth.device_packed_weights(2560, k, 95)     # [qkv 1024 | gate 768 | value 768]
    w2 = synth.device_packed_weights(1536, k, 96)     # FF-in: [gate 768 | value 768]
    w3 = synth.device_packed_weights(384, k, 97)      # plain
    W1, W2, W3 = (b1.device_weights(w1, k, 2560), b1.device_weights(w2, k, 1536),
                  b1.device_weights(w3, k, 384))
    p_out1 = torch.zeros(m * 1024 * 2, dtype=torch.uint8, device="cuda")    # [attn 256 | mlp 768]
    p_out2 = torch.zeros(m * 768 * 2, dtype=torch.uint8, device="cuda")
    qkv = torch.empty((m, 1024), device="cuda")
    y3 = torch.empty((m, 384), device="cuda")
    ops = [(a, W1, qkv, b1.packed_epilogue(1024, "swiglu", p_out1[256 * 2:], 1024)),
           (a, W3, y3),
           (a2, W2, None, b1.packed_epilogue(0, "swiglu", p_out2, 768))]
    b1.linear_batch(ops)
    torch.cuda.synchronize()
    p1_full = torch.zeros_like(p_out1)
    q_want, _ = b1.linear_packed_f16_to_packed(b1.pack_act_f16(a), w1, k, 2560, m, 1024, "swiglu",
                                               packed_out=p1_full[256 * 2:], ldp=1024)
    _, p2_want = b1.linear_packed_f16_to_packed(b1.pack_act_f16(a2), w2, k, 1536, m, 0, "swiglu")
    y3_want = b1.linear(a, w3, 384)
    torch.cuda.synchronize()
    assert torch.equal(qkv, q_want)
    assert torch.equal(p_out1, p1_full)
    assert torch.equal(p_out2, p2_want)
    assert torch.equal(y3, y3_want)
