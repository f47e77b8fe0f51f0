"""CPU oracle for the B1_0 1-bit linear -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or as the timed CPU baseline).
The product path (bonsai.cpp_amd/) never imports it.

Two layers:

* numpy restatements of the reference's Python side
    quantize_b1_0      convert_to_b1_0_packed.py:21-43
    dequantize_b1_0    tests/test_weight_parity.py:13-23
    dequant_unrounded  tests/c_ops/test_b1_linear.py:21-34 (fp32 mean, no
                       fp16 rounding -- the reference tests' own expectation)
    avx2_lane_model    lane-by-lane numpy model of src/b1_0_kernel.h:116-192
    norm_mod           ggml_norm + modulation of src/diffuser_graph.cpp:347-352
                       (ggml itself is not vendored: the definition is the
                       published LayerNorm, with the ggml CPU norm's double
                       accumulators; pinned by closed forms in the tests)
    swiglu_f64         silu(gate) * value over [gate | value]
                       (tests/ops/test_all_ops.py:29-45 of the reference;
                       pinned by closed forms and torch's silu)
    gelu_tanh_f64      0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), the
                       GELU-tanh between the C4 linears (a configuration
                       choice, not a reference op; pinned by torch's
                       gelu(approximate="tanh") and by erf-GELU closeness)
* ctypes bindings of the C restatement in b1_oracle.c (scalar spec path,
  AVX2 path with the reference tiling, fp64 brute force, pack/unpack,
  fp16 conversions).  Build it with `make -C oracle`.

How each function is pinned is listed in b1_oracle.h and tested in
tests/test_oracle.py.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

BLOCK_SIZE = 32
BLOCK_BYTES = 6

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libb1oracle.so"
_lib = None


# --------------------------------------------------------------- numpy ---

def quantize_b1_0(w: np.ndarray) -> np.ndarray:
    """fp32 [N, K] -> uint8 [N, K/32*6]; convert_to_b1_0_packed.py:21-43.

    scale = fp16(mean(|w|)) per 32-block, bit = (w >= 0), bytes
    [scale_lo, scale_hi, bits0, bits1, bits2, bits3].
    """
    n, k = w.shape
    assert k % BLOCK_SIZE == 0
    nb = k // BLOCK_SIZE
    r = w.reshape(n, nb, BLOCK_SIZE)
    scales = np.mean(np.abs(r), axis=-1).astype(np.float16)
    bits = (r >= 0).astype(np.uint8)
    packed_bits = np.packbits(bits, axis=-1, bitorder="little")
    raw = np.zeros((n, nb, BLOCK_BYTES), dtype=np.uint8)
    raw[:, :, 0:2] = scales.view(np.uint8).reshape(n, nb, 2)
    raw[:, :, 2:6] = packed_bits
    return raw.reshape(n, -1)


def dequantize_b1_0(raw: np.ndarray, n: int, k: int) -> np.ndarray:
    """uint8 packed -> fp32 [N, K]; tests/test_weight_parity.py:13-23."""
    nb = k // BLOCK_SIZE
    r = np.asarray(raw, dtype=np.uint8).reshape(n, nb, BLOCK_BYTES)
    lo = r[:, :, 0].astype(np.uint16)
    hi = r[:, :, 1].astype(np.uint16)
    scales = (lo | (hi << 8)).view(np.float16).astype(np.float32)
    bits = np.unpackbits(r[:, :, 2:6], axis=-1, bitorder="little").astype(np.float32)
    signs = 2.0 * bits - 1.0
    return (signs * scales[:, :, None]).reshape(n, k)


def dequant_unrounded(w: np.ndarray) -> np.ndarray:
    """+-mean|w| per block without fp16 rounding (the reference tests'
    expectation, tests/c_ops/test_b1_linear.py:21-34), vectorised."""
    n, k = w.shape
    r = w.reshape(n, k // BLOCK_SIZE, BLOCK_SIZE)
    scale = np.mean(np.abs(r), axis=-1, keepdims=True)
    return np.where(r >= 0, scale, -scale).reshape(n, k).astype(np.float32)


def linear_f64(act: np.ndarray, raw: np.ndarray, n: int) -> np.ndarray:
    """act [M, K] @ dequant(raw).T in float64."""
    k = act.shape[1]
    wd = dequantize_b1_0(raw, n, k).astype(np.float64)
    return act.astype(np.float64) @ wd.T


def avx2_lane_model(act: np.ndarray, raw: np.ndarray, n: int) -> np.ndarray:
    """Lane-by-lane fp32 model of the reference AVX2 loop for full 4-row
    tiles (src/b1_0_kernel.h:116-192): per block, lane l sums
    ((+-a[l] + +-a[8+l]) + (+-a[16+l] + +-a[24+l])), multiplies by the
    scale, adds to its accumulator; the 8 lanes are then reduced as
    ((s0+s4)+(s1+s5)) + ((s2+s6)+(s3+s7))."""
    m, k = act.shape
    nb = k // BLOCK_SIZE
    r = np.asarray(raw, dtype=np.uint8).reshape(n, nb, BLOCK_BYTES)
    scales = (r[:, :, 0].astype(np.uint16) | (r[:, :, 1].astype(np.uint16) << 8)).view(np.float16).astype(np.float32)
    bits = np.unpackbits(r[:, :, 2:6], axis=-1, bitorder="little").astype(bool)  # [n, nb, 32]
    a = act.astype(np.float32).reshape(m, nb, 4, 8)                  # [m, nb, j, l]
    sgn = np.where(bits, np.float32(1), np.float32(-1)).reshape(n, nb, 4, 8)
    acc = np.zeros((m, n, 8), dtype=np.float32)
    for b in range(nb):
        x = a[:, None, b, :, :] * sgn[None, :, b, :, :]                # exact +-a
        term = (x[:, :, 0] + x[:, :, 1]) + (x[:, :, 2] + x[:, :, 3])   # [m, n, 8]
        acc = acc + term * scales[None, :, b, None]
    v = acc[:, :, 0:4] + acc[:, :, 4:8]
    return ((v[:, :, 0] + v[:, :, 1]) + (v[:, :, 2] + v[:, :, 3])).astype(np.float32)


# ------------------------------------------------------------- C oracle ---

def norm_mod(x: np.ndarray, scale: np.ndarray, shift: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Per row of x [rows, H] (src/diffuser_graph.cpp:347-352):
    mean = fp32(sum_f64(x) / H); v = fp32(x - mean);
    var = fp32(sum_f64(fp32(v * v)) / H); rstd = fp32(1 / fp32(sqrt(fp32(var + eps))));
    n = fp32(v * rstd); out = fp32(fp32(n * fp32(scale + 1)) + shift)."""
    x = np.asarray(x, np.float32)
    f = np.float32
    h = x.shape[1]
    mean = (x.astype(np.float64).sum(axis=1) / h).astype(np.float32)[:, None]
    v = (x - mean).astype(np.float32)
    var = ((v * v).astype(np.float32).astype(np.float64).sum(axis=1) / h).astype(np.float32)[:, None]
    rstd = (f(1.0) / np.sqrt((var + f(eps)).astype(np.float32))).astype(np.float32)
    n = (v * rstd).astype(np.float32)
    t = (np.asarray(scale, np.float32) + f(1.0)).astype(np.float32)[None, :]
    return ((n * t).astype(np.float32) + np.asarray(shift, np.float32)[None, :]).astype(np.float32)


def norm_mod_f64(x: np.ndarray, scale: np.ndarray, shift: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """The same LayerNorm + modulation in float64 throughout."""
    x = np.asarray(x, np.float64)
    mean = x.mean(axis=1, keepdims=True)
    var = ((x - mean) ** 2).mean(axis=1, keepdims=True)
    return (x - mean) / np.sqrt(var + eps) * (np.asarray(scale, np.float64) + 1.0) + np.asarray(shift, np.float64)


def pack_act_words(a: np.ndarray) -> np.ndarray:
    """fp32 [rows, K] -> the packed fp16 activations as u32 [rows, K/2]:
    word 16 j + d = fp16(a[32 j + d]) | fp16(a[32 j + d + 16]) << 16 (RNE)."""
    rows, k = a.shape
    hb = fp32_to_fp16_bits(np.ascontiguousarray(a, np.float32)).reshape(rows, k // 32, 32).astype(np.uint32)
    return (hb[:, :, :16] | (hb[:, :, 16:] << 16)).reshape(rows, k // 2)


def gelu_tanh_f64(x: np.ndarray) -> np.ndarray:
    """GELU with the tanh approximation, in float64."""
    x = np.asarray(x, np.float64)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def swiglu_f64(y: np.ndarray) -> np.ndarray:
    """[gate | value] -> silu(gate) * value in float64."""
    y = np.asarray(y, np.float64)
    h = y.shape[1] // 2
    g = y[:, :h]
    return g / (1.0 + np.exp(-g)) * y[:, h:2 * h]


def build() -> None:
    """Compile the C restatement into oracle/_build/ (gcc, a few seconds)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(_LIB_PATH))
        f32p = ctypes.POINTER(ctypes.c_float)
        u8p = ctypes.POINTER(ctypes.c_uint8)
        u16p = ctypes.POINTER(ctypes.c_uint16)
        f64p = ctypes.POINTER(ctypes.c_double)
        i, i64 = ctypes.c_int, ctypes.c_int64
        L.b1o_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.b1o_fp16_to_fp32.restype = ctypes.c_float
        L.b1o_fp32_to_fp16.argtypes = [ctypes.c_float]
        L.b1o_fp32_to_fp16.restype = ctypes.c_uint16
        L.b1o_fp16_to_fp32_n.argtypes = [u16p, f32p, ctypes.c_size_t]
        L.b1o_pack.argtypes = [f32p, i, i, u8p]
        L.b1o_pack_seq.argtypes = [f32p, i, i, u8p]
        L.b1o_unpack.argtypes = [u8p, i, i, f32p]
        for fn in (L.b1o_linear_scalar_task, L.b1o_linear_avx2_task):
            fn.argtypes = [f32p, u8p, f32p, i, i, i, i, i]
            fn.restype = i64
        L.b1o_linear.argtypes = [f32p, u8p, f32p, i, i, i, i, i, i]
        L.b1o_linear.restype = i64
        L.b1o_linear_f64.argtypes = [f32p, u8p, f64p, i, i, i]
        L.b1o_has_avx2.restype = i
        _lib = L
    return _lib


def _p(a: np.ndarray, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def fp16_to_fp32_bits(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().b1o_fp16_to_fp32_n(_p(h, ctypes.c_uint16), _p(out, ctypes.c_float), h.size)
    return out


def fp32_to_fp16_bits(f: np.ndarray) -> np.ndarray:
    L = lib()
    f = np.ascontiguousarray(f, dtype=np.float32).ravel()
    return np.array([L.b1o_fp32_to_fp16(float(x)) for x in f], dtype=np.uint16)


def pack(w: np.ndarray, order: str = "numpy") -> np.ndarray:
    """B1_0 writer.  order 'numpy': convert_to_b1_0_packed.py's np.mean;
    'sequential': tests/c_ops/test_b1_linear.cpp's left-to-right sum."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    out = np.empty((n, k // BLOCK_SIZE * BLOCK_BYTES), dtype=np.uint8)
    fn = {"numpy": lib().b1o_pack, "sequential": lib().b1o_pack_seq}[order]
    fn(_p(w, ctypes.c_float), n, k, _p(out, ctypes.c_uint8))
    return out


def unpack(raw: np.ndarray, n: int, k: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    out = np.empty((n, k), dtype=np.float32)
    lib().b1o_unpack(_p(raw, ctypes.c_uint8), n, k, _p(out, ctypes.c_float))
    return out


def linear(act: np.ndarray, raw: np.ndarray, n: int, variant: str = "avx2",
           nth: int = 4, nthreads: int | None = None):
    """Runs the restated reference op.  Returns (out [M, N] fp32, count of
    non-finite outputs).  variant: 'scalar' (src/b1_0_kernel.h:240-287) or
    'avx2' (src/b1_0_kernel.h:79-239).  nth = ggml task count (the row split),
    nthreads = OS threads used to run those tasks."""
    act = np.ascontiguousarray(act, dtype=np.float32)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    m, k = act.shape
    assert raw.size == n * (k // BLOCK_SIZE) * BLOCK_BYTES
    out = np.empty((m, n), dtype=np.float32)
    v = {"scalar": 0, "avx2": 1}[variant]
    if nthreads is None:
        nthreads = min(nth, os.cpu_count() or 1)
    bad = lib().b1o_linear(_p(act, ctypes.c_float), _p(raw, ctypes.c_uint8),
                           _p(out, ctypes.c_float), m, k, n, nth, nthreads, v)
    if bad < 0:
        raise RuntimeError(f"oracle variant {variant} unavailable")
    return out, int(bad)


def linear_f64_c(act: np.ndarray, raw: np.ndarray, n: int) -> np.ndarray:
    act = np.ascontiguousarray(act, dtype=np.float32)
    raw = np.ascontiguousarray(raw, dtype=np.uint8)
    m, k = act.shape
    out = np.empty((m, n), dtype=np.float64)
    lib().b1o_linear_f64(_p(act, ctypes.c_float), _p(raw, ctypes.c_uint8),
                         _p(out, ctypes.c_double), m, k, n)
    return out
