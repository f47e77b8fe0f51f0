"""Host-side checks of the C ABI library (no GPU compute).

The library must load, export every function include/bonsai_b1.h declares,
keep the reference's struct layouts, and reject bad arguments before it
touches the device.
"""
import ctypes

import pytest

import bonsai_b1
from bonsai_b1 import capi


def test_library_exports_every_declared_symbol():
    lib = bonsai_b1.load()
    names = bonsai_b1.declared_symbols()
    assert len(names) >= 7
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/bonsai_b1.h but not exported"


def test_struct_layouts_match_reference():
    # B1LinearUserData {int magic; int in_dim; int out_dim;} src/b1_0_kernel.h:31-35
    assert ctypes.sizeof(capi.B1LinearUserData) == 12
    assert capi.B1LinearUserData.magic.offset == 0
    assert capi.MAGIC == 0x31423142


def test_version_and_status_strings():
    lib = bonsai_b1.load()
    assert lib.bonsai_b1_version() >= 100
    assert lib.bonsai_b1_status_string(0) == b"ok"
    assert lib.bonsai_b1_status_string(3) == b"non-finite output"
    assert lib.bonsai_b1_status_string(99) == b"unknown status"
    assert b"scratch" in lib.bonsai_b1_status_string(8)


def test_new_entries_reject_before_device():
    """The no-alloc, scaled and packed-with-workspace entries check their
    arguments before touching a device."""
    lib = bonsai_b1.load()
    fake = 0x10000
    assert lib.bonsai_b1_linear_f32_noalloc(fake, 64, fake, 63, 32, 1, fake, 32, 0, None, None) == capi.ERR_ARG
    assert lib.bonsai_b1_linear_f32_noalloc(fake, 64, fake, 64, 32, 1, fake, 32, 7, None, None) == capi.ERR_ARG
    # no row scales for a non-empty batch
    assert lib.bonsai_b1_pack_act_f16_scaled(fake, 384, 384, 4, fake, None, None) == capi.ERR_ARG
    assert lib.bonsai_b1_pack_act_f16_scaled(fake, 384, 384, 4, fake, fake + 2, None) == capi.ERR_ARG
    assert lib.bonsai_b1_linear_packed_f16_scaled(fake, None, fake, 384, 64, 4, fake, 64, None,
                                                  None) == capi.ERR_ARG
    # a misaligned caller workspace
    assert lib.bonsai_b1_linear_packed_f16_ws(fake, fake, 384, 64, 4, fake, 64, None, fake + 8, 1 << 20,
                                              None) == capi.ERR_ARG


@pytest.mark.parametrize("args", [
    # (lda, in_dim, out_dim, batch, ldo, mode)
    (64, 63, 32, 1, 32, 0),      # in_dim % 32 != 0 (reference precondition)
    (64, 0, 32, 1, 32, 0),       # empty in_dim
    (64, 64, 0, 1, 32, 0),       # empty out_dim
    (64, 64, 32, -1, 32, 0),     # negative batch
    (32, 64, 32, 1, 32, 0),      # lda < in_dim
    (64, 64, 32, 1, 16, 0),      # ldo < out_dim
    (64, 64, 32, 1, 32, 9),      # unknown mode
])
def test_bad_arguments_rejected_before_device(args):
    lda, k, n, m, ldo, mode = args
    lib = bonsai_b1.load()
    fake = 0x10000  # never dereferenced: validation precedes any device call
    st = lib.bonsai_b1_linear_f32(fake, lda, fake, k, n, m, fake, ldo, mode, None, None)
    assert st == capi.ERR_ARG


def test_null_pointers_rejected():
    lib = bonsai_b1.load()
    assert lib.bonsai_b1_linear_f32(None, 64, None, 64, 32, 1, None, 32, 0, None, None) == capi.ERR_ARG
    w = capi.B1WeightsC()
    assert lib.bonsai_b1_weights_upload(None, 0, 64, 32, None, ctypes.byref(w)) == capi.ERR_ARG
    # wrong byte count for the packed layout
    buf = (ctypes.c_uint8 * 10)()
    assert lib.bonsai_b1_weights_upload(buf, 10, 64, 32, None, ctypes.byref(w)) == capi.ERR_ARG
    assert lib.bonsai_b1_weights_free(None) == capi.ERR_ARG


def test_packed_act_bytes():
    lib = bonsai_b1.load()
    assert lib.bonsai_b1_packed_act_bytes(4096, 3072) == 4096 * 3072 * 2
    assert lib.bonsai_b1_packed_act_bytes(0, 3072) == 0
    assert lib.bonsai_b1_packed_act_bytes(8, 33) == 0


@pytest.mark.parametrize("args", [
    # (packed_ptr, in_dim, out_dim, batch, ldo)
    (0x10000, 3072 - 32, 64, 8, 64),   # in_dim % 384 != 0
    (0x10008, 3072, 64, 8, 64),        # packed activations not 16-byte aligned
    (0x10000, 3072, 64, 8, 32),        # ldo < out_dim
    (0x10000, 3072, 64, -1, 64),       # negative batch
])
def test_linear_packed_rejects_before_device(args):
    pa, k, n, m, ldo = args
    lib = bonsai_b1.load()
    fake = 0x10000
    assert lib.bonsai_b1_linear_packed_f16(pa, fake, k, n, m, fake, ldo, None, None) == capi.ERR_ARG


def test_pack_rejects_before_device():
    lib = bonsai_b1.load()
    fake = 0x10000
    assert lib.bonsai_b1_pack_act_f16(fake, 64, 48, 2, fake, None) == capi.ERR_ARG      # in_dim % 32
    assert lib.bonsai_b1_pack_act_f16(fake, 66, 64, 2, fake, None) == capi.ERR_ARG      # lda % 4
    assert lib.bonsai_b1_pack_act_f16(fake + 4, 64, 64, 2, fake, None) == capi.ERR_ARG  # act alignment
    assert lib.bonsai_b1_pack_act_f16(fake, 64, 64, 2, fake + 8, None) == capi.ERR_ARG  # packed alignment
    assert lib.bonsai_b1_pack_act_f16(None, 64, 64, 2, fake, None) == capi.ERR_ARG


def test_linear_batch_rejects_before_device():
    lib = bonsai_b1.load()
    assert lib.bonsai_b1_linear_batch(None, 1, 0, None, None, 0, None, None) == capi.ERR_ARG
    w = capi.B1WeightsC()
    w.data, w.in_dim, w.out_dim = 0x10000, 64, 32
    bad_w = capi.B1WeightsC()
    bad_w.data, bad_w.in_dim, bad_w.out_dim = 0x10000, 48, 32      # in_dim % 32 != 0
    ops = (capi.LinearOp * 2)()
    for i, ww in enumerate((w, bad_w)):
        ops[i].act, ops[i].lda, ops[i].w = 0x10000, 64, ctypes.pointer(ww)
        ops[i].out, ops[i].ldo, ops[i].batch = 0x10000, 32, 4
    bad = ctypes.c_int(-1)
    assert lib.bonsai_b1_linear_batch(ops, 2, 0, None, None, 0, ctypes.byref(bad), None) == capi.ERR_ARG
    assert bad.value == 1
    assert lib.bonsai_b1_linear_batch(ops, 1, 9, None, None, 0, None, None) == capi.ERR_ARG   # mode


def _epi(kind, gate=0, residual=0, ldr=0):
    return capi.Epilogue(kind, gate or None, residual or None, ldr)


@pytest.mark.parametrize("case", [
    # (epilogue, out_dim, ldo)
    ("swiglu_odd_h", 96, 48),          # H = 48, not a multiple of 32
    ("swiglu_ldo", 128, 63),           # ldo < H
    ("gate_no_res", 64, 64),           # gate-residual without a residual
    ("gate_ldr", 64, 64),              # ldr < out_dim
    ("res_overlap", 64, 64),           # residual overlapping out, not equal to it
    ("res_alias_ld", 64, 64),          # residual == out with another row stride
    ("kind", 64, 64),                  # unknown kind
])
def test_epilogue_rejected_before_device(case):
    """bonsai_b1_linear_epi_f32 / _packed_f16_epi check the epilogue against
    the linear's shape and buffers before touching the device."""
    name, n, ldo = case
    lib = bonsai_b1.load()
    out = 0x100000
    e = {"swiglu_odd_h": _epi(2), "swiglu_ldo": _epi(2),
         "gate_no_res": _epi(1, gate=0x200000),
         "gate_ldr": _epi(1, gate=0x200000, residual=0x300000, ldr=32),
         "res_overlap": _epi(1, gate=0x200000, residual=out + 64, ldr=64),
         "res_alias_ld": _epi(1, gate=0x200000, residual=out, ldr=128),
         "kind": _epi(7)}[name]
    m, k = 32, 384
    assert lib.bonsai_b1_linear_epi_f32(0x400000, k, 0x500000, k, n, m, out, ldo, ctypes.byref(e), 0, None,
                                        None, 0, None) == capi.ERR_ARG
    assert lib.bonsai_b1_linear_packed_f16_epi(0x400000, 0x500000, k, n, m, out, ldo, ctypes.byref(e), None,
                                               None) == capi.ERR_ARG


def r256(b):
    return (b + 255) // 256 * 256


def pack_area(m, k):
    """The range-safe packing: fp16 rows, then m fp32 row scales, each area
    rounded up to 256 bytes."""
    return r256(m * k * 2) + r256(m * 4)


def test_epilogue_workspace_bytes():
    """The larger of the range-safe packing (fused path) and the linear's
    fp32 output (separate epilogue pass); a plain small-batch linear needs
    nothing (the small-M kernel converts the activations itself)."""
    lib = bonsai_b1.load()
    assert lib.bonsai_b1_linear_epi_workspace_bytes(256, 3072, 6144, 2, 0) == max(pack_area(256, 3072),
                                                                                  256 * 6144 * 4)
    assert lib.bonsai_b1_linear_epi_workspace_bytes(256, 3072, 1024, 1, 0) == max(pack_area(256, 3072),
                                                                                  256 * 1024 * 4)
    assert lib.bonsai_b1_linear_epi_workspace_bytes(8, 3072, 1024, 0, 0) == 0
    assert lib.bonsai_b1_linear_epi_workspace_bytes(8, 3000, 1024, 1, 0) == 0   # in_dim % 32


def test_workspace_bytes_by_kernel():
    """What each kernel choice needs (no device here, so no split-K): the
    packed GEMM the range-safe packing; EXACT, the fused-conversion GEMM
    (K % 384 != 0) and the small-M kernel (which converts the activations
    itself) nothing."""
    lib = bonsai_b1.load()
    auto, exact, gemm, gemv = 0, 2, 3, 4
    assert lib.bonsai_b1_workspace_bytes(4096, 3072, 12288, auto) == pack_area(4096, 3072)
    assert lib.bonsai_b1_workspace_bytes(4096, 3072, 12288, exact) == 0
    assert lib.bonsai_b1_workspace_bytes(4096, 448, 128, gemm) == 0
    assert lib.bonsai_b1_workspace_bytes(8, 3072, 18432, auto) == 0
    assert lib.bonsai_b1_workspace_bytes(8, 3072, 18432, gemv) == 0
    assert lib.bonsai_b1_workspace_bytes(8, 3072, 18432, gemm) == pack_area(8, 3072)
    assert lib.bonsai_b1_workspace_bytes(8, 448, 64, auto) == 0
    assert lib.bonsai_b1_workspace_bytes(17, 3072, 64, gemv) == 0   # not a small-M batch
    assert lib.bonsai_b1_linear_packed_workspace_bytes(256, 3072, 3072) == 0   # no device: unsplit


def test_norm_mod_rejects_before_device():
    lib = bonsai_b1.load()
    f = 0x100000
    ok = (f, 3072, 3072, 4, f + 0x10000, f + 0x20000, ctypes.c_float(1e-6))
    assert lib.bonsai_b1_norm_mod_f32(f, 3072, 3000, 4, f, f, ctypes.c_float(1e-6), f, 3072, None) == capi.ERR_ARG  # H % 32
    assert lib.bonsai_b1_norm_mod_f32(f, 3070, 3072, 4, f, f, ctypes.c_float(1e-6), f, 3072, None) == capi.ERR_ARG  # ldx < H
    assert lib.bonsai_b1_norm_mod_f32(f + 4, 3072, 3072, 4, f, f, ctypes.c_float(1e-6), f, 3072, None) == capi.ERR_ARG
    assert lib.bonsai_b1_norm_mod_f32(*ok, f + 0x30000, 3071, None) == capi.ERR_ARG      # ldy < H
    assert lib.bonsai_b1_norm_mod_pack_f16(*ok, f + 8, None) == capi.ERR_ARG             # packed alignment
    assert lib.bonsai_b1_norm_mod_pack_f16(f, 3072, 3072, 4, None, f, ctypes.c_float(1e-6), f, None) == capi.ERR_ARG


def test_batch_epi_rejects_before_device():
    """bonsai_b1_linear_batch_epi checks every op's epilogue before touching
    the device: a SwiGLU op whose weights have an odd number of 32-row
    pairs is named by bad_op."""
    lib = bonsai_b1.load()
    w = capi.B1WeightsC()
    w.data, w.in_dim, w.out_dim = 0x10000, 64, 64
    bad_w = capi.B1WeightsC()
    bad_w.data, bad_w.in_dim, bad_w.out_dim = 0x10000, 64, 96     # 2H = 96: H % 32 != 0
    ops = (capi.LinearOpEpi * 2)()
    for i, ww in enumerate((w, bad_w)):
        ops[i].op.act, ops[i].op.lda, ops[i].op.w = 0x10000, 64, ctypes.pointer(ww)
        ops[i].op.out, ops[i].op.ldo, ops[i].op.batch = 0x100000, 64, 4
        ops[i].epi.kind = capi.EPILOGUES["swiglu"]
    bad = ctypes.c_int(-1)
    assert lib.bonsai_b1_linear_batch_epi(ops, 2, 0, None, None, 0, ctypes.byref(bad), None) == capi.ERR_ARG
    assert bad.value == 1


def test_strided_producers_reject_before_device():
    """The column-range producers check the packed row stride and the
    SwiGLU width before any launch (no device here)."""
    lib = bonsai_b1.load()
    f = 0x100000
    for fn in (lib.bonsai_b1_pack_act_f16_ld, lib.bonsai_b1_gelu_tanh_pack_f16_ld):
        assert fn(f, 3072, 3072, 4, f, 3000, None) == capi.ERR_ARG     # ldp < in_dim
        assert fn(f, 3072, 3072, 4, f, 15364, None) == capi.ERR_ARG    # rows not 16-byte aligned
        assert fn(f, 3072, 3072, 4, f + 8, 15360, None) == capi.ERR_ARG
        assert fn(None, 3072, 3072, 4, f, 15360, None) == capi.ERR_ARG
    sw = lib.bonsai_b1_swiglu_pack_f16_ld
    assert sw(f, 6144, 3000, 4, f, 3072, None) == capi.ERR_ARG          # hidden % 32
    assert sw(f, 6000, 3072, 4, f, 3072, None) == capi.ERR_ARG          # lda < 2 hidden
    assert sw(f, 6144, 3072, 4, f, 3064, None) == capi.ERR_ARG          # ldp < hidden
    assert sw(f, 6144, 3072, 4, f, 3076, None) == capi.ERR_ARG          # ldp % 8
    assert lib.bonsai_b1_swiglu_pack_f16(f, 6144, 3072, 4, None, None) == capi.ERR_ARG


def test_packed_output_linear_rejects_before_device():
    """bonsai_b1_linear_packed_f16_to_packed checks split, act, strides,
    alignment and overlap before any launch (no device here)."""
    lib = bonsai_b1.load()
    fn = lib.bonsai_b1_linear_packed_f16_to_packed
    a, w, o, p = 0x1000000, 0x2000000, 0x40000000, 0x80000000  # far apart
    M, K, N = 64, 3072, 21504
    ok = (a, w, K, N, M, o, 9216, 9216, 1, p, 15360, None, None)

    def call(**kw):
        args = list(ok)
        names = ["act_p", "w", "k", "n", "m", "out", "ldo", "split", "act", "pk", "ldp", "nf", "s"]
        for key, val in kw.items():
            args[names.index(key)] = val
        return fn(*args)

    assert call() == capi.ERR_DEVICE                     # valid: fails only at the device
    assert call(split=100) == capi.ERR_ARG               # split % 32
    assert call(split=N + 32) == capi.ERR_ARG
    assert call(act=3) == capi.ERR_ARG
    assert call(act=2, split=9248) == capi.ERR_ARG       # SwiGLU split % 64
    assert call(act=2, n=21536) == capi.ERR_ARG          # SwiGLU columns % 64
    assert call(ldp=15364) == capi.ERR_ARG               # ldp % 8
    assert call(ldp=12000) == capi.ERR_ARG               # ldp < packed columns
    assert call(act=2, ldp=6136) == capi.ERR_ARG         # SwiGLU: ldp < (N - split) / 2
    assert call(act=2, ldp=6144) == capi.ERR_DEVICE
    assert call(ldo=9000) == capi.ERR_ARG                # ldo < split
    assert call(ldo=9218) == capi.ERR_ARG                # ldo % 4
    assert call(out=o + 4) == capi.ERR_ARG               # out not 16-byte aligned
    assert call(pk=p + 8) == capi.ERR_ARG                # packed_out not 16-byte aligned
    assert call(out=None) == capi.ERR_ARG
    assert call(pk=None) == capi.ERR_ARG
    assert call(split=N, ldo=N, pk=None) == capi.ERR_DEVICE   # no packed columns
    assert call(split=0, out=None, ldp=N) == capi.ERR_DEVICE   # no fp32 columns
    assert call(pk=a + 64) == capi.ERR_ARG               # packed_out overlaps the input
    assert call(out=p) == capi.ERR_ARG                   # the outputs overlap
    assert call(k=3000) == capi.ERR_ARG                  # in_dim % 384


def test_epilogue_struct_layout():
    """bonsai_b1_epilogue: the packed-output fields follow the original four,
    whose offsets are unchanged (int kind; gate; residual; int64 ldr; int
    split; int act; packed; int64 ldp)."""
    E = capi.Epilogue
    assert (E.kind.offset, E.gate.offset, E.residual.offset, E.ldr.offset) == (0, 8, 16, 24)
    assert (E.split.offset, E.act.offset, E.packed.offset, E.ldp.offset) == (32, 36, 40, 48)
    assert ctypes.sizeof(E) == 56
    assert ctypes.sizeof(capi.LinearOpEpi) == ctypes.sizeof(capi.LinearOp) + 56


def test_packed_epilogue_rejected_before_device():
    """The packed-output epilogue of bonsai_b1_linear_epi_f32 and of a batch
    op is checked like bonsai_b1_linear_packed_f16_to_packed."""
    lib = bonsai_b1.load()
    act, w, out, pk = 0x1000000, 0x2000000, 0x40000000, 0x80000000
    m, k, n = 64, 3072, 2048

    def call(split=512, a=1, packed=pk, ldp=1536, o=out, ldo=512):
        e = capi.Epilogue(3, None, None, 0, split, a, packed, ldp)
        return lib.bonsai_b1_linear_epi_f32(act, k, w, k, n, m, o, ldo, ctypes.byref(e), 0, None, None, 0, None)

    assert call() == capi.ERR_DEVICE
    assert call(split=0, o=None, ldo=0, ldp=2048) == capi.ERR_DEVICE     # no fp32 columns: out may be NULL
    assert call(split=100) == capi.ERR_ARG
    assert call(a=5) == capi.ERR_ARG
    assert call(a=2, split=544) == capi.ERR_ARG                          # SwiGLU split % 64
    assert call(ldp=1500) == capi.ERR_ARG
    assert call(ldo=500) == capi.ERR_ARG
    assert call(packed=pk + 4) == capi.ERR_ARG
    assert call(packed=out + 64) == capi.ERR_ARG                         # outputs overlap
    assert call(o=None) == capi.ERR_ARG
