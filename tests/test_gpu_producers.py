"""GPU checks of the producers that write the packed fp16 activations of a
GEMM directly, into a column range of a wider packed matrix
(bonsai_b1_pack_act_f16_ld, bonsai_b1_gelu_tanh_pack_f16_ld,
bonsai_b1_swiglu_pack_f16_ld).

Bars (all bit for bit):
  * producers of adjacent column ranges build exactly the packing of the
    fp32 concatenation (the single-stream block's linear2 input,
    [attention output | MLP activation]);
  * the SwiGLU producer over a plain GEMM's output equals the packing of
    the SwiGLU epilogue's fp32 output (same fp32 arithmetic), and that
    packing equals the oracle's restatement of the layout.
"""
import sys

import numpy as np
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


@pytest.mark.parametrize("m,k1,k2", [(200, 96, 672), (37, 3072, 12288), (4608, 3072, 12288)])
def test_strided_producers_build_concatenated_input(torch, b1, m, k1, k2):
    from bonsai_b1 import synth
    say(f"concat producers m={m} k1={k1} k2={k2}")
    a1 = synth.device_activations(m, k1, 71)
    wide = synth.device_activations(m, k2 + 64, 72)
    a2 = wide[:, 32:32 + k2]                          # lda != k2, 128-byte offset
    k = k1 + k2
    buf = torch.full((m * k * 2,), 0xAB, dtype=torch.uint8, device="cuda")
    b1.pack_act_f16(a1, packed=buf, ldp=k)
    b1.gelu_tanh_pack_f16(a2, packed=buf[k1 * 2:], ldp=k)
    want = b1.pack_act_f16(torch.cat([a1, b1.gelu_tanh(a2.contiguous())], 1))
    torch.cuda.synchronize()
    assert torch.equal(buf, want[:buf.numel()])
    if m <= 200:
        # the GEMM over the built input equals the linear over the fp32 concatenation
        w = synth.device_packed_weights(384, k, 73)
        y = b1.linear_packed_f16(buf, w, k, 384, m)
        cat = torch.cat([a1, b1.gelu_tanh(a2.contiguous())], 1)
        # the fp32 entry, split along K as the packed entry splits
        yr = b1.linear(cat, w, 384)
        torch.cuda.synchronize()
        assert torch.equal(y, yr)


# (4600: the 128 x 512 kernel; 4608 and the Klein FF-in's 4096: the 16x16
# tile kernels, 144 x 384 and 128 x 384, the fused SwiGLU pairing each
# wave's 24 gates with their values)
@pytest.mark.parametrize("m,k,h", [(300, 1152, 768), (64, 384, 96), (4600, 3072, 9216), (4608, 3072, 9216),
                                   (4096, 3072, 9216)])
def test_swiglu_pack_matches_fused_epilogue(torch, b1, oracle, m, k, h):
    from bonsai_b1 import synth
    say(f"swiglu pack m={m} k={k} h={h}")
    a = synth.device_activations(m, k, 74)
    w = synth.device_packed_weights(2 * h, k, 75)
    pa = b1.pack_act_f16(a)
    # [gates | values], unsplit along K as the fused epilogue runs (a
    # workspace too small for split-K partials)
    y = b1.linear_packed_f16(pa, w, k, 2 * h, m, workspace=torch.empty(16, dtype=torch.uint8, device="cuda"))
    p1 = b1.swiglu_pack_f16(y)
    out = b1.linear_packed_f16_epi(pa, w, k, 2 * h, m, "swiglu")  # fp32 [m, h]
    p2 = b1.pack_act_f16(out)
    # into the second column range of a wider packed matrix
    ld = h + 3072
    buf = torch.zeros(m * ld * 2, dtype=torch.uint8, device="cuda")
    b1.swiglu_pack_f16(y, packed=buf[3072 * 2:], ldp=ld)
    torch.cuda.synchronize()
    assert torch.equal(p1, p2)
    got = buf.view(m, ld * 2)[:, 3072 * 2:].contiguous().reshape(-1)
    assert torch.equal(got, p1[:got.numel()])
    assert bool((buf.view(m, ld * 2)[:, :3072 * 2] == 0).all()), "columns before the range untouched"
    if m * h <= 300 * 768:
        words = oracle.pack_act_words(out.cpu().numpy())
        assert np.array_equal(p2.cpu().numpy().view(np.uint32).reshape(m, h // 2), words)
