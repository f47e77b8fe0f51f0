"""Weight residency from .safetensors (bonsai_b1_safetensors_info without a
device, bonsai_b1_weights_load_safetensors on the GPU).  Files are written
with the safetensors package, as convert_to_b1_0_packed.py writes them
(U8 [out_dim, in_dim/32*6])."""
import ctypes
import struct

import numpy as np
import pytest

import bonsai_b1
from bonsai_b1 import capi, synth

ERR_NOT_FOUND, ERR_FORMAT, ERR_IO = 5, 6, 7


def info(path, name):
    lib = bonsai_b1.load()
    lib.bonsai_b1_safetensors_info.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int),
                                               ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_uint64),
                                               ctypes.POINTER(ctypes.c_uint64)]
    k, n = ctypes.c_int(), ctypes.c_int()
    off, nb = ctypes.c_uint64(), ctypes.c_uint64()
    st = lib.bonsai_b1_safetensors_info(str(path).encode(), name.encode(), ctypes.byref(k), ctypes.byref(n),
                                        ctypes.byref(off), ctypes.byref(nb))
    return st, k.value, n.value, off.value, nb.value


@pytest.fixture
def model_file(tmp_path):
    from safetensors.numpy import save_file
    tensors = {
        "transformer_blocks.0.attn.to_q.weight": synth.packed_weights(48, 256, 1),
        "single_transformer_blocks.3.proj_out.weight": synth.packed_weights(8, 3072, 2),
        "norm.weight": np.ones((3, 4), np.float32),
        "odd": np.zeros((5, 7), np.uint8),
        "café \"q\"": synth.packed_weights(2, 64, 3),
    }
    path = tmp_path / "model.safetensors"
    save_file(tensors, str(path), metadata={"format": "b1_0"})
    return path, tensors


def test_info_locates_b1_tensors(model_file):
    path, tensors = model_file
    blob = path.read_bytes()
    for name, k, n in [("transformer_blocks.0.attn.to_q.weight", 256, 48),
                       ("single_transformer_blocks.3.proj_out.weight", 3072, 8),
                       ("café \"q\"", 64, 2)]:
        st, kk, nn, off, nb = info(path, name)
        assert st == 0, name
        assert (kk, nn) == (k, n)
        assert nb == n * k // 32 * 6
        assert blob[off:off + nb] == tensors[name].tobytes()


def test_info_errors(model_file, tmp_path):
    path, _ = model_file
    assert info(path, "missing")[0] == ERR_NOT_FOUND
    assert info(path, "norm.weight")[0] == ERR_FORMAT          # F32, not a B1_0 tensor
    assert info(path, "odd")[0] == ERR_FORMAT                  # 7 bytes per row
    assert info(tmp_path / "nope.safetensors", "x")[0] == ERR_IO
    blob = path.read_bytes()
    import json
    hlen = struct.unpack("<Q", blob[:8])[0]
    entries = {k: v for k, v in json.loads(blob[8:8 + hlen]).items() if k != "__metadata__"}
    last = max(entries, key=lambda k: entries[k]["data_offsets"][1])
    first = min(entries, key=lambda k: entries[k]["data_offsets"][1])
    (tmp_path / "trunc.safetensors").write_bytes(blob[:-10])    # data cut short
    assert info(tmp_path / "trunc.safetensors", last)[0] == ERR_FORMAT
    if first != last and entries[first]["dtype"] == "U8" and entries[first]["shape"][1] % 6 == 0:
        assert info(tmp_path / "trunc.safetensors", first)[0] == 0   # earlier tensors are intact
    (tmp_path / "tiny.safetensors").write_bytes(b"\x01\x02")
    assert info(tmp_path / "tiny.safetensors", "x")[0] == ERR_FORMAT
    hdr = b'{"w": {"dtype": "U8", "shape": [1, 6], "data_offsets": [0, 6]}'   # unterminated object
    (tmp_path / "bad.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(6))
    assert info(tmp_path / "bad.safetensors", "w")[0] == ERR_FORMAT
    hdr = b'{"w": {"dtype": "U8", "shape": [2, 6], "data_offsets": [0, 6]}}'  # shape says 12 bytes
    (tmp_path / "short.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(6))
    assert info(tmp_path / "short.safetensors", "w")[0] == ERR_FORMAT
    (tmp_path / "huge.safetensors").write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    assert info(tmp_path / "huge.safetensors", "w")[0] == ERR_FORMAT


@pytest.mark.gpu
def test_load_uploads_and_runs(model_file, oracle):
    import torch
    path, tensors = model_file
    name = "transformer_blocks.0.attn.to_q.weight"
    lib = bonsai_b1.load()
    lib.bonsai_b1_weights_load_safetensors.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_void_p,
                                                       ctypes.POINTER(capi.B1WeightsC)]
    w = capi.B1WeightsC()
    st = lib.bonsai_b1_weights_load_safetensors(str(path).encode(), name.encode(),
                                                ctypes.c_void_p(torch.cuda.current_stream().cuda_stream),
                                                ctypes.byref(w))
    assert st == 0
    assert (w.in_dim, w.out_dim, w.nbytes) == (256, 48, 48 * 8 * 6)
    import glob
    import os
    hip_path = sorted(glob.glob(os.path.join(os.path.dirname(torch.__file__), "lib", "libamdhip64.so*")))[0]
    hip = ctypes.CDLL(hip_path)                 # the runtime torch already loaded
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    dev = torch.empty(w.nbytes, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    assert hip.hipMemcpy(dev.data_ptr(), w.data, w.nbytes, 3) == 0   # hipMemcpyDeviceToDevice
    torch.cuda.synchronize()
    assert np.array_equal(dev.cpu().numpy(), tensors[name].ravel())
    act = synth.activations(5, 256, 9)
    y = bonsai_b1.linear(torch.from_numpy(act).cuda(), dev, 48, mode="exact")
    torch.cuda.synchronize()
    want, _ = oracle.linear(act, tensors[name], 48, variant="scalar")
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
    assert lib.bonsai_b1_weights_free(ctypes.byref(w)) == 0


# --------------------------------------------- the open-file handle (CPU) --

def test_open_enumerates_and_finds(model_file):
    path, tensors = model_file
    with bonsai_b1.SafetensorsFile(path) as f:
        names = f.names()
        assert sorted(names) == sorted(tensors)            # every tensor, B1_0 or not
        lib = bonsai_b1.load()
        assert lib.bonsai_b1_safetensors_name(f._h, len(names)) is None
        assert lib.bonsai_b1_safetensors_name(f._h, -1) is None
        for name in ("transformer_blocks.0.attn.to_q.weight", "single_transformer_blocks.3.proj_out.weight",
                     "café \"q\""):
            st, k, n, off, nb = info(path, name)
            assert st == 0
            assert f.find(name) == (k, n, off, nb)
        for name, code in (("missing", ERR_NOT_FOUND), ("norm.weight", ERR_FORMAT), ("odd", ERR_FORMAT)):
            with pytest.raises(bonsai_b1.B1Error) as e:
                f.find(name)
            assert e.value.status == code


def test_open_errors(tmp_path):
    def open_status(p):
        h = ctypes.c_void_p()
        return bonsai_b1.load().bonsai_b1_safetensors_open(str(p).encode(), ctypes.byref(h)), h
    st, h = open_status(tmp_path / "nope.safetensors")
    assert st == ERR_IO and not h.value
    (tmp_path / "tiny.safetensors").write_bytes(b"\x01\x02")
    assert open_status(tmp_path / "tiny.safetensors")[0] == ERR_FORMAT
    hdr = b'{"w": {"dtype": "U8", "shape": [1, 6], "data_offsets": [0, 6]}, "w": {"dtype": "U8"}}'  # repeated
    (tmp_path / "dup.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(6))
    assert open_status(tmp_path / "dup.safetensors")[0] == ERR_FORMAT
    hdr = b'{"__metadata__": {"a": "b"}, "w": {"dtype": "U8", "shape": [1, 6], "data_offsets": [0, 6]}}'
    (tmp_path / "meta.safetensors").write_bytes(struct.pack("<Q", len(hdr)) + hdr + bytes(6))
    with bonsai_b1.SafetensorsFile(tmp_path / "meta.safetensors") as f:
        assert f.names() == ["w"]                           # metadata is not a tensor
        assert f.find("w")[:2] == (32, 1)


def test_load_checks_every_name_before_the_device(model_file):
    """Bad names fail before anything is allocated (no device needed), and
    out[] stays zeroed."""
    path, _ = model_file
    lib = bonsai_b1.load()
    with bonsai_b1.SafetensorsFile(path) as f:
        for bad, code in ((["transformer_blocks.0.attn.to_q.weight", "missing"], ERR_NOT_FOUND),
                          (["norm.weight"], ERR_FORMAT)):
            arr = (ctypes.c_char_p * len(bad))(*[n.encode() for n in bad])
            out = (capi.B1WeightsC * len(bad))()
            assert lib.bonsai_b1_safetensors_load(f._h, arr, len(bad), None, out) == code
            assert all(not out[i].data and out[i].nbytes == 0 for i in range(len(bad)))
        assert lib.bonsai_b1_safetensors_load(f._h, None, 0, None, None) == 0
        assert lib.bonsai_b1_safetensors_load(None, None, 0, None, None) == 1
        assert lib.bonsai_b1_safetensors_load(f._h, None, 1, None, None) == 1


# ------------------------------------------------ pinned pipeline (GPU) --

@pytest.mark.gpu
def test_handle_loads_many_tensors_through_staging(tmp_path):
    """One call uploads several tensors, one of them larger than a staging
    buffer (16 MB), so pieces go round all three buffers and each buffer is
    refilled after its copy completes; every device byte equals the file's."""
    import torch
    from safetensors.numpy import save_file
    tensors = {
        "big": synth.packed_weights(12288, 12288, 21),       # 28.3 MB: two pieces
        "a": synth.packed_weights(3072, 3072, 22),           # 1.8 MB
        "b": synth.packed_weights(96, 512, 23),
        "c": synth.packed_weights(9216, 3072, 24),           # 5.3 MB
        "d": synth.packed_weights(18432, 3072, 25),          # 10.6 MB
    }
    path = tmp_path / "many.safetensors"
    save_file(tensors, str(path))
    order = ["b", "big", "a", "d", "c"]
    with bonsai_b1.SafetensorsFile(path) as f:
        ws = f.load(order)
        ws2 = f.load(["a"])                                  # the handle's buffers are reused
    try:
        for name, w in zip(order + ["a"], ws + ws2):
            host = tensors[name]
            assert (w.out_dim, w.in_dim, w.nbytes) == (host.shape[0], host.shape[1] // 6 * 32, host.nbytes)
            dev = torch.empty(w.nbytes, dtype=torch.uint8, device="cuda")
            torch.cuda.synchronize()
            import glob
            import os
            hip = ctypes.CDLL(sorted(glob.glob(os.path.join(os.path.dirname(torch.__file__), "lib",
                                                            "libamdhip64.so*")))[0])
            hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
            assert hip.hipMemcpy(dev.data_ptr(), w.data, w.nbytes, 3) == 0
            torch.cuda.synchronize()
            assert np.array_equal(dev.cpu().numpy(), host.ravel()), name
    finally:
        for w in ws + ws2:
            bonsai_b1.weights_free(w)
