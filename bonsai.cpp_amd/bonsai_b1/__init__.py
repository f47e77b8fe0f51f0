"""Python plumbing over the gfx950 B1_0 linear C ABI (include/bonsai_b1.h).

The compute lives in lib/libbonsai_b1.so (HIP kernels for gfx950); this
module only passes torch device pointers and the current torch stream to it
through ctypes.  There is no CPU fallback: if the library is missing or the
device is not gfx950, calls raise.
"""
from .capi import (  # noqa: F401
    B1Error,
    MODES,
    SafetensorsFile,
    Weights,
    weights_free,
    declared_symbols,
    device_weights,
    linear_batch,
    linear_batch_workspace_bytes,
    linear_epi,
    linear_epi_workspace_bytes,
    norm_mod,
    linear_packed_f16_epi,
    linear_packed_f16_to_packed,
    packed_epilogue,
    ACTS,
    EPILOGUES,
    gelu_tanh,
    gelu_tanh_pack_f16,
    library_path,
    linear,
    linear_packed_f16,
    linear_packed_f16_scaled,
    pack_act_f16_scaled,
    linear_packed_workspace_bytes,
    linear_raw,
    load,
    pack_act_f16,
    quantize_f32,
    swiglu_pack_f16,
    workspace_bytes,
)
from . import synth  # noqa: F401
