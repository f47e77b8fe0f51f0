"""Seeded synthetic inputs of the benchmark recipe.

Activations ~ N(0,1) fp32; packed B1_0 weights with sign words of
independent Bernoulli(0.5) bits and fp16 scales fp16(U[lo, hi]).
Host generation uses numpy's PCG64 (deterministic for a seed); device
generation uses torch's generator on the GPU (for the large benchmark
tensors).
"""
from __future__ import annotations

import numpy as np

BLOCK_SIZE = 32
BLOCK_BYTES = 6


def activations(m: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal((m, k), dtype=np.float32)


def packed_weights(n: int, k: int, seed: int, lo: float = 0.005, hi: float = 0.05) -> np.ndarray:
    """uint8 [n, k/32*6] in the convert_to_b1_0_packed.py layout."""
    assert k % BLOCK_SIZE == 0
    nb = k // BLOCK_SIZE
    rng = np.random.Generator(np.random.PCG64(seed))
    words = rng.integers(0, 1 << 32, size=(n, nb), dtype=np.uint32)
    scale = (lo + (hi - lo) * rng.random((n, nb))).astype(np.float16)
    raw = np.empty((n, nb, BLOCK_BYTES), dtype=np.uint8)
    raw[:, :, 0:2] = scale.astype("<f2").view(np.uint8).reshape(n, nb, 2)
    raw[:, :, 2:6] = words.astype("<u4").view(np.uint8).reshape(n, nb, 4)
    return raw.reshape(n, nb * BLOCK_BYTES)


def device_activations(m: int, k: int, seed: int, device="cuda"):
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return torch.randn((m, k), generator=g, device=device, dtype=torch.float32)


def device_packed_weights(n: int, k: int, seed: int, lo: float = 0.005, hi: float = 0.05, device="cuda"):
    """uint8 cuda tensor [n, k/32*6], same layout and distribution."""
    import torch
    nb = k // BLOCK_SIZE
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    raw = torch.randint(0, 256, (n, nb, BLOCK_BYTES), generator=g, device=device, dtype=torch.uint8)
    u = torch.rand((n, nb), generator=g, device=device, dtype=torch.float32)
    scale = (lo + (hi - lo) * u).to(torch.float16)
    raw[:, :, 0:2] = scale.view(torch.uint8).reshape(n, nb, 2)
    return raw.reshape(n, nb * BLOCK_BYTES)
