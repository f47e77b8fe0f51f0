"""Writes / loads the committed golden fixtures for the B1_0 linear.

Each fixture holds seeded inputs (activations, packed weights in the
convert_to_b1_0_packed.py layout) and the outputs of the oracle's scalar
path (src/b1_0_kernel.h:240-287 order), its AVX2 path (:79-239 order, 4 ggml
tasks) and the fp64 brute force.  Regenerate with
    python tests/golden/make_golden.py
(numpy .npz, arrays only; loaded with allow_pickle=False).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent

# name: (M, K, N, seed_a, seed_w)
CASES = {
    "ref_shape_m1_k64_n32": (1, 64, 32, 101, 102),
    "ragged_m5_k256_n40": (5, 256, 40, 103, 104),
    "gemv_m8_k3072_n48": (8, 3072, 48, 105, 106),
    "gemm_m160_k192_n72": (160, 192, 72, 107, 108),
    "odd_blocks_m3_k96_n16": (3, 96, 16, 109, 110),
    "gemm_m200_k384_n600": (200, 384, 600, 111, 112),
}


def load_all() -> dict:
    out = {}
    for name in CASES:
        p = HERE / f"{name}.npz"
        if p.exists():
            with np.load(p, allow_pickle=False) as z:
                out[name] = {k: z[k] for k in z.files}
    return out


def main() -> None:
    for p in (ROOT, ROOT / "bonsai.cpp_amd"):
        sys.path.insert(0, str(p))
    from bonsai_b1 import synth
    from oracle import b1_oracle as o
    for name, (m, k, n, sa, sw) in CASES.items():
        act = synth.activations(m, k, sa)
        w = synth.packed_weights(n, k, sw)
        ys, bad1 = o.linear(act, w, n, variant="scalar", nth=4)
        ya, bad2 = o.linear(act, w, n, variant="avx2", nth=4)
        assert bad1 == 0 and bad2 == 0
        yf = o.linear_f64(act, w, n)
        np.savez(HERE / f"{name}.npz", act=act, w=w, n=np.int64(n), seed_a=np.int64(sa),
                 seed_w=np.int64(sw), y_scalar=ys, y_avx2=ya, y_f64=yf)
        print(f"wrote {name}.npz")


if __name__ == "__main__":
    main()
