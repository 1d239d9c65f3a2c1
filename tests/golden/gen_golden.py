"""Writes the golden activation-quantization vectors from the reference's own code.

Runs only in a container where the reference tree is mounted: it builds
oracle/_ref/libnsos_ref.so from OXN/nsos/src/bitlinear_quantize_avx2.cpp
(oracle/Makefile target `ref`) and records that library's outputs for seeded
and constructed inputs.  The fixtures are data (inputs and expected outputs);
the GPU box and CPU tests read them without the reference.

    python tests/golden/gen_golden.py
"""
from __future__ import annotations

import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402


def tie_rows() -> np.ndarray:
    """Rows whose scaled values land exactly on .5 ties.

    With max|x| = 127, s = 127/(127 + 1e-8f) = 1.0f, so x*s = x: entries k+0.5
    are exact ties.  19 columns = 16-column AVX2 body + 3-column scalar tail.
    """
    base = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 3.5,
                     4.5, -4.5, 5.5, 6.5, -6.5, 7.5, 0.25, -0.75,
                     0.5, 2.5, -1.5], np.float32)
    alt = base.copy()
    alt[0] = -127.0
    alt[16:] = [1.5, -0.5, 126.5]
    return np.stack([base, alt])


def main() -> None:
    oracle.build()
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref not built: the reference tree is not mounted here")
    rng = np.random.default_rng(20261201)
    cases = {
        "c1_16x768": rng.standard_normal((16, 768)).astype(np.float32),
        "tail_5x1003": (rng.standard_normal((5, 1003)) * 3.0).astype(np.float32),
        "ties_2x19": tie_rows(),
        "small_3x7": rng.standard_normal((3, 7)).astype(np.float32),
    }
    out = {}
    for name, x in cases.items():
        out[f"{name}__x"] = x
        for bits in (2, 4, 8):
            codes, scales = oracle.ref_quantize_rows(x, bits)
            assert np.all(codes == np.round(codes))
            out[f"{name}__b{bits}__codes"] = codes.astype(np.int16)
            out[f"{name}__b{bits}__scales"] = scales
    w = rng.integers(-1, 2, size=(6, 1000)).astype(np.int8)
    out["rowsum__w"] = w
    out["rowsum__sums"] = np.array([oracle.ref_row_sum_i8(r) for r in w], np.int32)
    path = os.path.join(HERE, "quant_ref.npz")
    np.savez_compressed(path, **out)
    digest = hashlib.sha256(open(path, "rb").read()).hexdigest()
    with open(os.path.join(HERE, "MANIFEST.sha256"), "w") as fh:
        fh.write(f"{digest}  quant_ref.npz\n")
    print(f"wrote {path} sha256={digest}")


if __name__ == "__main__":
    main()
