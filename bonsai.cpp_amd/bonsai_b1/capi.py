"""ctypes binding of libbonsai_b1.so (declarations in include/bonsai_b1.h)."""
from __future__ import annotations

import ctypes
import os
import re
from pathlib import Path

_PKG = Path(__file__).resolve().parent.parent          # bonsai.cpp_amd/
_REPO = _PKG.parent
# BONSAI_B1_LIB names another build of the same library (the host-sanitized
# one of `make -C bonsai.cpp_amd sanitize`); by default the in-tree build.
_LIB = Path(os.environ["BONSAI_B1_LIB"]).resolve() if os.environ.get("BONSAI_B1_LIB") else \
    _PKG / "lib" / "libbonsai_b1.so"
_HDR = _REPO / "include" / "bonsai_b1.h"

BLOCK_SIZE = 32
BLOCK_BYTES = 6
MAGIC = 0x31423142

OK, ERR_ARG, ERR_HIP, ERR_NONFINITE, ERR_DEVICE = 0, 1, 2, 3, 4
ERR_SCRATCH = 8
# bytes of the static device workspace of bonsai_b1_linear_f32_noalloc
NOALLOC_SCRATCH_BYTES = 32 << 20
MODES = {"auto": 0, "fast": 1, "exact": 2, "gemm": 3, "gemv": 4}

_lib = None


class B1Error(RuntimeError):
    def __init__(self, status: int, what: str = ""):
        self.status = status
        text = load().bonsai_b1_status_string(status).decode()
        super().__init__(f"{what}: {text} (status {status})" if what else text)


class B1LinearUserData(ctypes.Structure):
    _fields_ = [("magic", ctypes.c_int), ("in_dim", ctypes.c_int), ("out_dim", ctypes.c_int)]


class B1WeightsC(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("in_dim", ctypes.c_int), ("out_dim", ctypes.c_int),
                ("nbytes", ctypes.c_size_t), ("device", ctypes.c_int)]


EPILOGUES = {"none": 0, "gate_residual": 1, "swiglu": 2, "packed": 3}
ACTS = {"none": 0, "gelu_tanh": 1, "swiglu": 2}


class Epilogue(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("gate", ctypes.c_void_p), ("residual", ctypes.c_void_p),
                ("ldr", ctypes.c_int64), ("split", ctypes.c_int), ("act", ctypes.c_int),
                ("packed", ctypes.c_void_p), ("ldp", ctypes.c_int64)]


class LinearOp(ctypes.Structure):
    _fields_ = [("act", ctypes.c_void_p), ("lda", ctypes.c_int64), ("w", ctypes.POINTER(B1WeightsC)),
                ("out", ctypes.c_void_p), ("ldo", ctypes.c_int64), ("batch", ctypes.c_int)]


class LinearOpEpi(ctypes.Structure):
    _fields_ = [("op", LinearOp), ("epi", Epilogue)]


def library_path() -> Path:
    return _LIB


def declared_symbols() -> list[str]:
    """Every extern "C" function declared in include/bonsai_b1.h."""
    text = _HDR.read_text()
    return sorted(set(re.findall(r"^\w[\w\s\*]*?\b(bonsai_b1_\w+)\s*\(", text, re.M)))


def load():
    """Load the HIP library (torch first, so both share one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    import torch  # noqa: F401  -- loads torch's libamdhip64 before ours
    if not _LIB.exists():
        raise FileNotFoundError(f"{_LIB} is not built; run __graft_entry__.build() or make -C bonsai.cpp_amd")
    L = ctypes.CDLL(str(_LIB))
    vp, i, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    L.bonsai_b1_linear_f32.argtypes = [vp, i64, vp, i, i, i, vp, i64, i, vp, vp]
    L.bonsai_b1_linear_f32.restype = i
    L.bonsai_b1_linear_f32_ws.argtypes = [vp, i64, vp, i, i, i, vp, i64, i, vp, vp, ctypes.c_size_t, vp]
    L.bonsai_b1_linear_f32_ws.restype = i
    L.bonsai_b1_linear_f32_noalloc.argtypes = [vp, i64, vp, i, i, i, vp, i64, i, vp, vp]
    L.bonsai_b1_linear_f32_noalloc.restype = i
    L.bonsai_b1_workspace_bytes.argtypes = [i, i, i, i]
    L.bonsai_b1_workspace_bytes.restype = ctypes.c_size_t
    L.bonsai_b1_linear.argtypes = [vp, ctypes.POINTER(B1WeightsC), i, vp,
                                   ctypes.POINTER(B1LinearUserData), i, vp, vp]
    L.bonsai_b1_linear.restype = i
    L.bonsai_b1_weights_upload.argtypes = [vp, ctypes.c_size_t, i, i, vp, ctypes.POINTER(B1WeightsC)]
    L.bonsai_b1_weights_upload.restype = i
    L.bonsai_b1_weights_free.argtypes = [ctypes.POINTER(B1WeightsC)]
    L.bonsai_b1_weights_free.restype = i
    L.bonsai_b1_status_string.argtypes = [i]
    L.bonsai_b1_status_string.restype = ctypes.c_char_p
    L.bonsai_b1_version.restype = i
    L.bonsai_b1_linear_f32_f32.argtypes = [vp, i, i, vp]
    L.bonsai_b1_linear_f32_f32.restype = None
    L.bonsai_b1_callback_defer.argtypes = [i]
    L.bonsai_b1_callback_defer.restype = i
    L.bonsai_b1_callback_finish.argtypes = [ctypes.POINTER(ctypes.c_int32)]
    L.bonsai_b1_callback_finish.restype = i
    L.bonsai_b1_linear_batch.argtypes = [ctypes.POINTER(LinearOp), i, i, vp, vp, ctypes.c_size_t,
                                         ctypes.POINTER(i), vp]
    L.bonsai_b1_linear_batch.restype = i
    L.bonsai_b1_linear_batch_workspace_bytes.argtypes = [ctypes.POINTER(LinearOp), i, i]
    L.bonsai_b1_linear_batch_workspace_bytes.restype = ctypes.c_size_t
    L.bonsai_b1_gelu_tanh_f32.argtypes = [vp, i64, vp, i64, i, i, vp]
    L.bonsai_b1_gelu_tanh_f32.restype = i
    L.bonsai_b1_gelu_tanh_pack_f16.argtypes = [vp, i64, i, i, vp, vp]
    L.bonsai_b1_gelu_tanh_pack_f16.restype = i
    L.bonsai_b1_gelu_tanh_pack_f16_ld.argtypes = [vp, i64, i, i, vp, i64, vp]
    L.bonsai_b1_gelu_tanh_pack_f16_ld.restype = i
    L.bonsai_b1_swiglu_pack_f16.argtypes = [vp, i64, i, i, vp, vp]
    L.bonsai_b1_swiglu_pack_f16.restype = i
    L.bonsai_b1_swiglu_pack_f16_ld.argtypes = [vp, i64, i, i, vp, i64, vp]
    L.bonsai_b1_swiglu_pack_f16_ld.restype = i
    L.bonsai_b1_quantize_f32.argtypes = [vp, i64, i, i, vp, i, vp]
    L.bonsai_b1_quantize_f32.restype = i
    L.bonsai_b1_packed_act_bytes.argtypes = [i, i]
    L.bonsai_b1_packed_act_bytes.restype = ctypes.c_size_t
    L.bonsai_b1_pack_act_f16.argtypes = [vp, i64, i, i, vp, vp]
    L.bonsai_b1_pack_act_f16.restype = i
    L.bonsai_b1_pack_act_f16_ld.argtypes = [vp, i64, i, i, vp, i64, vp]
    L.bonsai_b1_pack_act_f16_ld.restype = i
    L.bonsai_b1_linear_packed_f16.argtypes = [vp, vp, i, i, i, vp, i64, vp, vp]
    L.bonsai_b1_linear_packed_f16.restype = i
    L.bonsai_b1_linear_packed_f16_ws.argtypes = [vp, vp, i, i, i, vp, i64, vp, vp, ctypes.c_size_t, vp]
    L.bonsai_b1_linear_packed_f16_ws.restype = i
    L.bonsai_b1_pack_act_f16_scaled.argtypes = [vp, i64, i, i, vp, vp, vp]
    L.bonsai_b1_pack_act_f16_scaled.restype = i
    L.bonsai_b1_linear_packed_f16_scaled.argtypes = [vp, vp, vp, i, i, i, vp, i64, vp, vp]
    L.bonsai_b1_linear_packed_f16_scaled.restype = i
    L.bonsai_b1_linear_packed_workspace_bytes.argtypes = [i, i, i]
    L.bonsai_b1_linear_packed_workspace_bytes.restype = ctypes.c_size_t
    L.bonsai_b1_linear_packed_f16_epi.argtypes = [vp, vp, i, i, i, vp, i64, ctypes.POINTER(Epilogue), vp, vp]
    L.bonsai_b1_linear_packed_f16_epi.restype = i
    L.bonsai_b1_linear_packed_f16_to_packed.argtypes = [vp, vp, i, i, i, vp, i64, i, i, vp, i64, vp, vp]
    L.bonsai_b1_linear_packed_f16_to_packed.restype = i
    L.bonsai_b1_linear_epi_workspace_bytes.argtypes = [i, i, i, i, i]
    L.bonsai_b1_linear_epi_workspace_bytes.restype = ctypes.c_size_t
    L.bonsai_b1_linear_epi_f32.argtypes = [vp, i64, vp, i, i, i, vp, i64, ctypes.POINTER(Epilogue), i, vp, vp,
                                           ctypes.c_size_t, vp]
    L.bonsai_b1_linear_epi_f32.restype = i
    L.bonsai_b1_linear_batch_epi.argtypes = [ctypes.POINTER(LinearOpEpi), i, i, vp, vp, ctypes.c_size_t,
                                             ctypes.POINTER(i), vp]
    L.bonsai_b1_linear_batch_epi.restype = i
    L.bonsai_b1_linear_batch_epi_workspace_bytes.argtypes = [ctypes.POINTER(LinearOpEpi), i, i]
    L.bonsai_b1_linear_batch_epi_workspace_bytes.restype = ctypes.c_size_t
    L.bonsai_b1_weights_concat.argtypes = [ctypes.POINTER(B1WeightsC), i, vp, ctypes.POINTER(B1WeightsC)]
    L.bonsai_b1_weights_concat.restype = i
    L.bonsai_b1_norm_mod_f32.argtypes = [vp, i64, i, i, vp, vp, ctypes.c_float, vp, i64, vp]
    L.bonsai_b1_norm_mod_f32.restype = i
    L.bonsai_b1_norm_mod_pack_f16.argtypes = [vp, i64, i, i, vp, vp, ctypes.c_float, vp, vp]
    L.bonsai_b1_norm_mod_pack_f16.restype = i
    L.bonsai_b1_safetensors_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(vp)]
    L.bonsai_b1_safetensors_open.restype = i
    L.bonsai_b1_safetensors_close.argtypes = [vp]
    L.bonsai_b1_safetensors_close.restype = None
    L.bonsai_b1_safetensors_count.argtypes = [vp]
    L.bonsai_b1_safetensors_count.restype = i
    L.bonsai_b1_safetensors_name.argtypes = [vp, i]
    L.bonsai_b1_safetensors_name.restype = ctypes.c_char_p
    L.bonsai_b1_safetensors_find.argtypes = [vp, ctypes.c_char_p, ctypes.POINTER(i), ctypes.POINTER(i),
                                             ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]
    L.bonsai_b1_safetensors_find.restype = i
    L.bonsai_b1_safetensors_load.argtypes = [vp, ctypes.POINTER(ctypes.c_char_p), i, vp,
                                             ctypes.POINTER(B1WeightsC)]
    L.bonsai_b1_safetensors_load.restype = i
    _lib = L
    return L


def _stream_handle(stream):
    import torch
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def linear_raw(act_ptr: int, lda: int, w_ptr: int, in_dim: int, out_dim: int, batch: int,
               out_ptr: int, ldo: int, mode: str = "auto", nonfinite_ptr: int = 0,
               stream_handle: int = 0) -> int:
    """Direct call with raw device pointers; returns the status code."""
    return load().bonsai_b1_linear_f32(act_ptr, lda, w_ptr, in_dim, out_dim, batch, out_ptr, ldo,
                                       MODES[mode], nonfinite_ptr or None, stream_handle or None)


def workspace_bytes(batch: int, in_dim: int, out_dim: int, mode: str = "auto") -> int:
    return int(load().bonsai_b1_workspace_bytes(batch, in_dim, out_dim, MODES[mode]))


def linear(act, w_packed, out_dim: int, out=None, mode: str = "auto", nonfinite=None, stream=None,
           workspace=None):
    """out[M, N] = B1_0 linear of act[M, K] (fp32, cuda, row stride >= K)
    with packed weights w_packed (uint8, cuda, N*(K/32)*6 bytes).
    Returns `out` (allocated if None).  Stream-ordered; does not sync.
    With `workspace` (a cuda tensor) the caller's buffer replaces the
    library-owned one (bonsai_b1_linear_f32_ws; never allocates)."""
    import torch
    if act.dim() != 2 or act.dtype != torch.float32 or not act.is_cuda or act.stride(1) != 1:
        raise ValueError("act must be a 2-D fp32 cuda tensor with unit column stride")
    m, k = act.shape
    if w_packed.dtype != torch.uint8 or not w_packed.is_cuda or not w_packed.is_contiguous():
        raise ValueError("w_packed must be a contiguous uint8 cuda tensor")
    if w_packed.numel() != out_dim * (k // BLOCK_SIZE) * BLOCK_BYTES:
        raise ValueError("w_packed size does not match out_dim * in_dim/32 * 6")
    if out is None:
        out = torch.empty((m, out_dim), dtype=torch.float32, device=act.device)
    if out.dim() != 2 or out.shape[0] != m or out.shape[1] < out_dim or out.stride(1) != 1:
        raise ValueError("out must be [M, >=N] fp32 with unit column stride")
    nf = nonfinite.data_ptr() if nonfinite is not None else None
    if workspace is not None:
        st = load().bonsai_b1_linear_f32_ws(act.data_ptr(), act.stride(0), w_packed.data_ptr(), k, out_dim, m,
                                            out.data_ptr(), out.stride(0), MODES[mode], nf, workspace.data_ptr(),
                                            workspace.numel() * workspace.element_size(), _stream_handle(stream))
    else:
        st = load().bonsai_b1_linear_f32(act.data_ptr(), act.stride(0), w_packed.data_ptr(), k, out_dim, m,
                                         out.data_ptr(), out.stride(0), MODES[mode], nf, _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_linear_f32")
    return out


def gelu_tanh(x, out=None, stream=None):
    """GELU-tanh of a 2-D fp32 cuda tensor (bonsai_b1_gelu_tanh_f32); out may be x."""
    import torch
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda or x.stride(1) != 1:
        raise ValueError("x must be a 2-D fp32 cuda tensor with unit column stride")
    if out is None:
        out = torch.empty_like(x)
    rows, cols = x.shape
    st = load().bonsai_b1_gelu_tanh_f32(x.data_ptr(), x.stride(0), out.data_ptr(), out.stride(0), cols, rows,
                                        _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_gelu_tanh_f32")
    return out


def _packed_target(act, packed, ldp):
    """The packed buffer of a producer: new when None; with ldp (packed row
    length in fp16 elements) a view starting at the target column range."""
    import torch
    m, k = act.shape
    if ldp is None:
        nbytes = load().bonsai_b1_packed_act_bytes(m, k)
        if packed is None:
            packed = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=act.device)
        if packed.numel() < nbytes or not packed.is_contiguous():
            raise ValueError("packed must hold bonsai_b1_packed_act_bytes(M, K) contiguous bytes")
    elif packed is None or packed.numel() < ((m - 1) * ldp + k) * 2 or not packed.is_contiguous():
        raise ValueError("packed must be a contiguous view holding (M-1)*ldp + K fp16 elements")
    return packed


def gelu_tanh_pack_f16(act, packed=None, stream=None, ldp=None):
    """Packed fp16 activations of gelu_tanh(act) (bonsai_b1_gelu_tanh_pack_f16;
    with ldp, bonsai_b1_gelu_tanh_pack_f16_ld into a column range)."""
    m, k = act.shape
    packed = _packed_target(act, packed, ldp)
    if ldp is None:
        st = load().bonsai_b1_gelu_tanh_pack_f16(act.data_ptr(), act.stride(0), k, m, packed.data_ptr(),
                                                 _stream_handle(stream))
    else:
        st = load().bonsai_b1_gelu_tanh_pack_f16_ld(act.data_ptr(), act.stride(0), k, m, packed.data_ptr(), ldp,
                                                    _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_gelu_tanh_pack_f16")
    return packed


def swiglu_pack_f16(act, packed=None, stream=None, ldp=None):
    """Packed fp16 activations of SwiGLU over act [M, 2H] (gates first):
    silu(a[:, :H]) * a[:, H:] (bonsai_b1_swiglu_pack_f16; with ldp,
    bonsai_b1_swiglu_pack_f16_ld into the column range `packed` starts at)."""
    import torch
    m, k2 = act.shape
    if k2 % 2:
        raise ValueError("act must hold 2H columns")
    h = k2 // 2
    if ldp is None:
        if packed is None:
            packed = torch.empty(max(m * h * 2, 16), dtype=torch.uint8, device=act.device)
        st = load().bonsai_b1_swiglu_pack_f16(act.data_ptr(), act.stride(0), h, m, packed.data_ptr(),
                                              _stream_handle(stream))
    else:
        if packed is None or packed.numel() < ((m - 1) * ldp + h) * 2:
            raise ValueError("packed must be a view holding (M-1)*ldp + H fp16 elements")
        st = load().bonsai_b1_swiglu_pack_f16_ld(act.data_ptr(), act.stride(0), h, m, packed.data_ptr(), ldp,
                                                 _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_swiglu_pack_f16")
    return packed


def device_weights(w_packed, in_dim: int, out_dim: int) -> B1WeightsC:
    """A B1Weights view of packed weights already in a cuda tensor (the
    tensor must outlive the view)."""
    c = B1WeightsC()
    c.data = w_packed.data_ptr()
    c.in_dim, c.out_dim = in_dim, out_dim
    c.nbytes = w_packed.numel()
    c.device = w_packed.device.index or 0
    return c


def _batch_ops(ops):
    with_epi = any(len(op) > 3 for op in ops)
    arr = ((LinearOpEpi if with_epi else LinearOp) * len(ops))()
    keep = []
    for i, op in enumerate(ops):
        act, w, out = op[:3]
        keep.append(w)
        o = arr[i].op if with_epi else arr[i]
        o.act, o.lda = act.data_ptr(), act.stride(0)
        o.w = ctypes.pointer(w)
        o.out, o.ldo = (out.data_ptr(), out.stride(0)) if out is not None else (None, 0)
        o.batch = act.shape[0]
        if with_epi:
            spec = op[3] if len(op) > 3 else "none"
            if isinstance(spec, Epilogue):
                arr[i].epi = spec
            elif isinstance(spec, str):
                arr[i].epi = _epilogue(spec, None, None, w.out_dim, act.shape[0])
            else:
                arr[i].epi = _epilogue(spec[0], spec[1], spec[2], w.out_dim, act.shape[0])
    return arr, with_epi, keep


def linear_batch_workspace_bytes(ops, mode: str = "auto") -> int:
    """Workspace bytes a linear_batch call over `ops` uses on the current
    device (bonsai_b1_linear_batch[_epi]_workspace_bytes)."""
    arr, with_epi, _ = _batch_ops(ops)
    fn = load().bonsai_b1_linear_batch_epi_workspace_bytes if with_epi else \
        load().bonsai_b1_linear_batch_workspace_bytes
    return int(fn(arr, len(ops), MODES[mode]))


def linear_batch(ops, mode: str = "auto", nonfinite=None, workspace=None, stream=None):
    """bonsai_b1_linear_batch over [(act, B1WeightsC, out), ...] (cuda
    tensors, act/out 2-D fp32 with unit column stride).  An op may carry a
    fourth item, its epilogue: "swiglu", ("gate_residual", gate,
    residual) or a packed_epilogue() (then out holds the split fp32
    columns, or is None when split == 0); then bonsai_b1_linear_batch_epi
    runs the list."""
    arr, with_epi, keep = _batch_ops(ops)
    bad = ctypes.c_int(-1)
    nf = nonfinite.data_ptr() if nonfinite is not None else None
    ws = workspace.data_ptr() if workspace is not None else None
    wsb = workspace.numel() * workspace.element_size() if workspace is not None else 0
    fn = load().bonsai_b1_linear_batch_epi if with_epi else load().bonsai_b1_linear_batch
    st = fn(arr, len(ops), MODES[mode], nf, ws, wsb, ctypes.byref(bad), _stream_handle(stream))
    if st != OK:
        raise B1Error(st, f"bonsai_b1_linear_batch (op {bad.value})")


SUM_ORDERS = {"numpy": 0, "sequential": 1}


def quantize_f32(w, order: str = "numpy", out=None, stream=None):
    """Packed B1_0 bytes (uint8 cuda [N, K/32*6]) of fp32 cuda weights w[N, K]
    (bonsai_b1_quantize_f32)."""
    import torch
    if w.dim() != 2 or w.dtype != torch.float32 or not w.is_cuda or w.stride(1) != 1:
        raise ValueError("w must be a 2-D fp32 cuda tensor with unit column stride")
    n, k = w.shape
    if out is None:
        out = torch.empty((n, k // BLOCK_SIZE * BLOCK_BYTES), dtype=torch.uint8, device=w.device)
    st = load().bonsai_b1_quantize_f32(w.data_ptr(), w.stride(0), k, n, out.data_ptr(), SUM_ORDERS[order],
                                       _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_quantize_f32")
    return out


def pack_act_f16(act, packed=None, stream=None, ldp=None):
    """fp16 K-slot-paired activations of act[M, K] (bonsai_b1_pack_act_f16);
    returns a uint8 cuda tensor of M*K*2 bytes.  With ldp (packed row length
    in fp16 elements), bonsai_b1_pack_act_f16_ld into the column range that
    the `packed` view starts at."""
    import torch
    if act.dim() != 2 or act.dtype != torch.float32 or not act.is_cuda or act.stride(1) != 1:
        raise ValueError("act must be a 2-D fp32 cuda tensor with unit column stride")
    m, k = act.shape
    packed = _packed_target(act, packed, ldp)
    if ldp is None:
        st = load().bonsai_b1_pack_act_f16(act.data_ptr(), act.stride(0), k, m, packed.data_ptr(),
                                           _stream_handle(stream))
    else:
        st = load().bonsai_b1_pack_act_f16_ld(act.data_ptr(), act.stride(0), k, m, packed.data_ptr(), ldp,
                                              _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_pack_act_f16")
    return packed


def pack_act_f16_scaled(act, packed=None, row_scale=None, stream=None):
    """Range-safe packing (bonsai_b1_pack_act_f16_scaled): returns (packed
    uint8 [M*K*2], row_scale fp32 [M])."""
    import torch
    if act.dim() != 2 or act.dtype != torch.float32 or not act.is_cuda or act.stride(1) != 1:
        raise ValueError("act must be a 2-D fp32 cuda tensor with unit column stride")
    m, k = act.shape
    packed = _packed_target(act, packed, None)
    if row_scale is None:
        row_scale = torch.empty(m, dtype=torch.float32, device=act.device)
    st = load().bonsai_b1_pack_act_f16_scaled(act.data_ptr(), act.stride(0), k, m, packed.data_ptr(),
                                              row_scale.data_ptr(), _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_pack_act_f16_scaled")
    return packed, row_scale


def linear_packed_f16_scaled(packed, row_scale, w_packed, in_dim: int, out_dim: int, batch: int, out=None,
                             nonfinite=None, stream=None):
    """bonsai_b1_linear_packed_f16_scaled: the packed linear with row m's
    outputs multiplied by row_scale[m]."""
    import torch
    if out is None:
        out = torch.empty((batch, out_dim), dtype=torch.float32, device=packed.device)
    if out.dim() != 2 or out.shape[0] != batch or out.shape[1] < out_dim or out.stride(1) != 1:
        raise ValueError("out must be [batch, >=out_dim] fp32 with unit column stride")
    nf = nonfinite.data_ptr() if nonfinite is not None else None
    st = load().bonsai_b1_linear_packed_f16_scaled(packed.data_ptr(), row_scale.data_ptr(), w_packed.data_ptr(),
                                                   in_dim, out_dim, batch, out.data_ptr(), out.stride(0), nf,
                                                   _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_linear_packed_f16_scaled")
    return out


def linear_packed_workspace_bytes(batch: int, in_dim: int, out_dim: int) -> int:
    return int(load().bonsai_b1_linear_packed_workspace_bytes(batch, in_dim, out_dim))


def linear_packed_f16(packed, w_packed, in_dim: int, out_dim: int, batch: int, out=None, nonfinite=None,
                      stream=None, workspace=None):
    """out[batch, out_dim] from packed fp16 activations (bonsai_b1_linear_packed_f16;
    with `workspace`, a cuda tensor, bonsai_b1_linear_packed_f16_ws)."""
    import torch
    if out is None:
        out = torch.empty((batch, out_dim), dtype=torch.float32, device=packed.device)
    if out.dim() != 2 or out.shape[0] != batch or out.shape[1] < out_dim or out.stride(1) != 1:
        raise ValueError("out must be [batch, >=out_dim] fp32 with unit column stride")
    nf = nonfinite.data_ptr() if nonfinite is not None else None
    if workspace is not None:
        st = load().bonsai_b1_linear_packed_f16_ws(packed.data_ptr(), w_packed.data_ptr(), in_dim, out_dim, batch,
                                                   out.data_ptr(), out.stride(0), nf, workspace.data_ptr(),
                                                   workspace.numel() * workspace.element_size(),
                                                   _stream_handle(stream))
    else:
        st = load().bonsai_b1_linear_packed_f16(packed.data_ptr(), w_packed.data_ptr(), in_dim, out_dim, batch,
                                                out.data_ptr(), out.stride(0), nf, _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_linear_packed_f16")
    return out


def _epilogue(kind: str, gate, residual, n_out: int, m: int):
    """The C epilogue struct for `kind`, checking the tensors' shapes."""
    import torch
    e = Epilogue(EPILOGUES[kind], None, None, 0)
    if kind == "gate_residual":
        if gate is None or residual is None:
            raise ValueError("gate_residual needs gate [N] and residual [M, >=N]")
        for t in (gate, residual):
            if t.dtype != torch.float32 or not t.is_cuda or t.stride(-1) != 1:
                raise ValueError("gate and residual must be fp32 cuda tensors with unit column stride")
        if gate.numel() < n_out or residual.dim() != 2 or residual.shape[0] != m or residual.shape[1] < n_out:
            raise ValueError("gate must have N entries and residual shape [M, >=N]")
        e.gate, e.residual, e.ldr = gate.data_ptr(), residual.data_ptr(), residual.stride(0)
    return e


def packed_epilogue(split: int, act: str, packed, ldp: int):
    """The BONSAI_B1_EPI_PACKED epilogue: y columns [0, split) stay fp32 in
    the op's out, columns [split, N) go through `act` ("none", "gelu_tanh",
    "swiglu") into the packed fp16 activations `packed` (a uint8 cuda view
    starting at the target column, rows of ldp fp16 elements)."""
    return Epilogue(EPILOGUES["packed"], None, None, 0, split, ACTS[act],
                    packed.data_ptr() if packed is not None else None, ldp)


def linear_epi_workspace_bytes(batch: int, in_dim: int, out_dim: int, epilogue: str, mode: str = "auto") -> int:
    return int(load().bonsai_b1_linear_epi_workspace_bytes(batch, in_dim, out_dim, EPILOGUES[epilogue],
                                                            MODES[mode]))


def linear_epi(act, w_packed, out_dim: int, epilogue: str, gate=None, residual=None, out=None,
               mode: str = "auto", nonfinite=None, workspace=None, stream=None):
    """The linear with a fused epilogue (bonsai_b1_linear_epi_f32):
    "gate_residual" -> out = residual + gate * y (residual may be out);
    "swiglu" -> out[:, j] = silu(y[:, j]) * y[:, H + j], H = out_dim / 2;
    or a packed_epilogue(): out [M, >=split] (None when split == 0) and the
    epilogue's packed fp16 output.  Returns out."""
    import torch
    m, k = act.shape
    if isinstance(epilogue, Epilogue):     # packed_epilogue(): out holds the split fp32 columns
        e, cols = epilogue, epilogue.split
    else:
        e, cols = _epilogue(epilogue, gate, residual, out_dim, m), (out_dim // 2 if epilogue == "swiglu"
                                                                   else out_dim)
    if out is None and cols > 0:
        out = torch.empty((m, cols), dtype=torch.float32, device=act.device)
    if out is not None and (out.dim() != 2 or out.shape[0] != m or out.shape[1] < cols or out.stride(1) != 1):
        raise ValueError("out must be [M, >=cols] fp32 with unit column stride")
    nf = nonfinite.data_ptr() if nonfinite is not None else None
    ws, wsb = (workspace.data_ptr(), workspace.numel() * workspace.element_size()) if workspace is not None \
        else (None, 0)
    st = load().bonsai_b1_linear_epi_f32(act.data_ptr(), act.stride(0), w_packed.data_ptr(), k, out_dim, m,
                                         out.data_ptr() if out is not None else None,
                                         out.stride(0) if out is not None else 0, ctypes.byref(e), MODES[mode],
                                         nf, ws, wsb, _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_linear_epi_f32")
    return out


def linear_packed_f16_epi(packed, w_packed, in_dim: int, out_dim: int, batch: int, epilogue: str, gate=None,
                          residual=None, out=None, nonfinite=None, stream=None):
    """bonsai_b1_linear_packed_f16_epi: the packed GEMM with its epilogue fused."""
    import torch
    cols = out_dim // 2 if epilogue == "swiglu" else out_dim
    if out is None:
        out = torch.empty((batch, cols), dtype=torch.float32, device=packed.device)
    if out.dim() != 2 or out.shape[0] != batch or out.shape[1] < cols or out.stride(1) != 1:
        raise ValueError("out must be [batch, >=cols] fp32 with unit column stride")
    e = _epilogue(epilogue, gate, residual, out_dim, batch)
    nf = nonfinite.data_ptr() if nonfinite is not None else None
    st = load().bonsai_b1_linear_packed_f16_epi(packed.data_ptr(), w_packed.data_ptr(), in_dim, out_dim, batch,
                                                out.data_ptr(), out.stride(0), ctypes.byref(e), nf,
                                                _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_linear_packed_f16_epi")
    return out


def linear_packed_f16_to_packed(packed, w_packed, in_dim: int, out_dim: int, batch: int, split: int,
                                act: str = "none", out=None, packed_out=None, ldp=None, nonfinite=None,
                                stream=None):
    """bonsai_b1_linear_packed_f16_to_packed: y columns [0, split) as fp32
    into out [batch, >=split]; columns [split, out_dim) through `act`
    ("none", "gelu_tanh", or "swiglu" over [gate | value]) into packed fp16
    activations: a new [batch, cols] packing when packed_out is None,
    otherwise packed_out (contiguous; with ldp, a view starting at the
    target column range of rows of ldp fp16 elements).  Returns (out,
    packed_out); out is None when split == 0."""
    import torch
    cols = (out_dim - split) // 2 if act == "swiglu" else out_dim - split
    if out is None and split > 0:
        out = torch.empty((batch, split), dtype=torch.float32, device=packed.device)
    if out is not None and (out.dim() != 2 or out.shape[0] != batch or out.shape[1] < split or out.stride(1) != 1):
        raise ValueError("out must be [batch, >=split] fp32 with unit column stride")
    if ldp is None:
        ldp = cols
        if packed_out is None and cols > 0:
            packed_out = torch.empty(max(batch * cols * 2, 16), dtype=torch.uint8, device=packed.device)
    if cols > 0 and (packed_out is None or not packed_out.is_contiguous()
                     or packed_out.numel() * packed_out.element_size() < ((batch - 1) * ldp + cols) * 2):
        raise ValueError("packed_out must be a contiguous view holding (batch-1)*ldp + cols fp16 elements")
    nf = nonfinite.data_ptr() if nonfinite is not None else None
    st = load().bonsai_b1_linear_packed_f16_to_packed(
        packed.data_ptr(), w_packed.data_ptr(), in_dim, out_dim, batch,
        out.data_ptr() if out is not None else None, out.stride(0) if out is not None else 0, split, ACTS[act],
        packed_out.data_ptr() if packed_out is not None else None, ldp, nf, _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_linear_packed_f16_to_packed")
    return out, packed_out


def norm_mod(x, scale, shift, eps: float = 1e-6, out=None, packed=None, stream=None):
    """LayerNorm (no affine) + modulation x_n * (scale + 1) + shift over the
    rows of x [rows, H]: fp32 into `out`, or, with packed=True or a uint8
    tensor, the packed fp16 activations (bonsai_b1_norm_mod_pack_f16)."""
    import torch
    rows, h = x.shape
    if packed is not None:
        if packed is True:
            packed = torch.empty(rows * h * 2, dtype=torch.uint8, device=x.device)
        st = load().bonsai_b1_norm_mod_pack_f16(x.data_ptr(), x.stride(0), h, rows, scale.data_ptr(),
                                                shift.data_ptr(), eps, packed.data_ptr(), _stream_handle(stream))
        if st != OK:
            raise B1Error(st, "bonsai_b1_norm_mod_pack_f16")
        return packed
    if out is None:
        out = torch.empty((rows, h), dtype=torch.float32, device=x.device)
    st = load().bonsai_b1_norm_mod_f32(x.data_ptr(), x.stride(0), h, rows, scale.data_ptr(), shift.data_ptr(), eps,
                                       out.data_ptr(), out.stride(0), _stream_handle(stream))
    if st != OK:
        raise B1Error(st, "bonsai_b1_norm_mod_f32")
    return out


class SafetensorsFile:
    """An open .safetensors file (bonsai_b1_safetensors_open): mapped and its
    header parsed once, like bonsai::SafetensorsFile (src/safetensors.h:
    27-90).  load() makes B1_0 tensors device-resident through the pinned
    staging pipeline (bonsai_b1_safetensors_load)."""

    def __init__(self, path):
        h = ctypes.c_void_p()
        st = load().bonsai_b1_safetensors_open(str(path).encode(), ctypes.byref(h))
        if st != OK:
            raise B1Error(st, "bonsai_b1_safetensors_open")
        self._h = h

    def names(self):
        L = load()
        return [L.bonsai_b1_safetensors_name(self._h, i).decode()
                for i in range(L.bonsai_b1_safetensors_count(self._h))]

    def find(self, name: str):
        """(in_dim, out_dim, data_offset, nbytes) of B1_0 tensor `name`."""
        k, n = ctypes.c_int(), ctypes.c_int()
        off, nb = ctypes.c_uint64(), ctypes.c_uint64()
        st = load().bonsai_b1_safetensors_find(self._h, name.encode(), ctypes.byref(k), ctypes.byref(n),
                                               ctypes.byref(off), ctypes.byref(nb))
        if st != OK:
            raise B1Error(st, "bonsai_b1_safetensors_find")
        return k.value, n.value, off.value, nb.value

    def load(self, names, stream=None):
        """B1WeightsC for each name (free each with weights_free).  stream:
        a torch stream, a raw handle (int), or None for the current one."""
        arr = (ctypes.c_char_p * max(1, len(names)))(*[n.encode() for n in names])
        out = (B1WeightsC * max(1, len(names)))()
        sh = ctypes.c_void_p(stream) if isinstance(stream, int) else _stream_handle(stream)
        st = load().bonsai_b1_safetensors_load(self._h, arr, len(names), sh, out)
        if st != OK:
            raise B1Error(st, "bonsai_b1_safetensors_load")
        return [out[i] for i in range(len(names))]

    def close(self):
        if self._h:
            load().bonsai_b1_safetensors_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def weights_free(w):
    """bonsai_b1_weights_free on a B1WeightsC."""
    st = load().bonsai_b1_weights_free(ctypes.byref(w))
    if st != OK:
        raise B1Error(st, "bonsai_b1_weights_free")


class Weights:
    """Device-resident packed weights via bonsai_b1_weights_upload."""

    def __init__(self, host_packed, in_dim: int, out_dim: int, stream=None):
        import numpy as np
        self._host = np.ascontiguousarray(host_packed, dtype=np.uint8)
        self.c = B1WeightsC()
        st = load().bonsai_b1_weights_upload(self._host.ctypes.data, self._host.nbytes, in_dim, out_dim,
                                             _stream_handle(stream), ctypes.byref(self.c))
        if st != OK:
            raise B1Error(st, "bonsai_b1_weights_upload")

    @property
    def in_dim(self):
        return self.c.in_dim

    @property
    def out_dim(self):
        return self.c.out_dim

    def linear(self, act, out=None, mode: str = "auto", nonfinite=None, stream=None, ud=None):
        import torch
        m = act.shape[0]
        if out is None:
            out = torch.empty((m, self.out_dim), dtype=torch.float32, device=act.device)
        if ud is None:
            ud = B1LinearUserData()
        nf = nonfinite.data_ptr() if nonfinite is not None else None
        st = load().bonsai_b1_linear(act.data_ptr(), ctypes.byref(self.c), m, out.data_ptr(), ctypes.byref(ud),
                                     MODES[mode], nf, _stream_handle(stream))
        if st != OK:
            raise B1Error(st, "bonsai_b1_linear")
        return out

    def free(self):
        if self.c.data:
            st = load().bonsai_b1_weights_free(ctypes.byref(self.c))
            if st != OK:
                raise B1Error(st, "bonsai_b1_weights_free")

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass
