"""GPU checks of the GEMM epilogue that writes the next linear's packed fp16
activations (bonsai_b1_linear_packed_f16_to_packed).

Bar (bit for bit): the fp32 columns equal the plain GEMM's output (the same
128-row tile, the same K order), and the packed columns equal the packing
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
]


@pytest.mark.parametrize("m,k,n,split,act,col0,ldp", CASES)
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
