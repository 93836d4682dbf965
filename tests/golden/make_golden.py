"""Writes tests/golden/exl3_golden.npz: small fixtures that freeze the oracle's
decode (codebook LUT digests, one-tile windows and weights per bit width, and a
tiny dense linear).  The reference ships no golden vectors for this path, so the
fixtures are generated from the oracle after the checks in tests/test_oracle.py
(reference host helper, numpy IEEE arithmetic, fragment layout) pinned it.
Run from the repo root: python tests/golden/make_golden.py"""

import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from dsv4_carve_amd import synth  # noqa: E402


def main():
    out = {}
    for cb in (0, 1, 2):
        out[f"lut_sha256_cb{cb}"] = np.array(hashlib.sha256(O.codebook_lut(cb).tobytes()).hexdigest())
    rng = np.random.default_rng(20261201)
    for bits in (2, 3, 4, 6):
        tr = rng.integers(0, 1 << 16, (1, 1, 16 * bits), dtype=np.uint16).view(np.int16)
        out[f"tile_trellis_k{bits}"] = tr
        out[f"tile_windows_k{bits}"] = O.windows_np(tr, bits)
        out[f"tile_wq_k{bits}"] = O.reconstruct_c(tr, bits).view(np.uint16)
    L = synth.dense(128, 256, 3, seed=99)
    x = synth.activations(2, 128, seed=99)
    out.update(dense_x=x, dense_trellis=L["trellis"], dense_suh=L["suh"], dense_svh=L["svh"],
               dense_bits=np.array(3), dense_y=O.linear(x, L["trellis"], L["suh"], L["svh"], 3))
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "exl3_golden.npz")
    np.savez_compressed(path, **out)
    print("wrote", path, os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
