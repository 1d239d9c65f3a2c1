"""Writes golden vectors from the reference's own compiled code.

Runs only in a container where the reference tree is mounted: it builds
oracle/_ref/libnsos_ref.so from the reference's sources (oracle/Makefile
target `ref`: the AVX2 quantizer, Tensor, BitLinear and the files their link
needs) and records that library's outputs for seeded and constructed inputs:

  quant_ref.npz      the AVX2 activation quantizer and weight row sums
  tensor_ref.npz     Tensor::rmsnorm / softmax / silu / silu_gate /
                     squared_relu / rmsnorm_backward, tensor_abs_mean, and the
                     RMS_PERI int8 codes of BitLinear::forward's quantizer
  bitlinear_ref.npz  BitLinear::forward (packed ternary and float paths) and
                     the packed STE backward
  mamba2_ref.npz     Mamba2SSD::forward on the faithful Mamba-2 path, the
                     non-sensitive projections packed ternary
  mamba2_n64_ref.npz the same at the reference's default state width
                     (mamba_d_state 64) with head_dim 64 and two groups

Inputs are stored as float16-representable values (cast to float32 before
use) so the fixtures stay small.  The fixtures are data (inputs and expected
outputs); the GPU box and CPU tests read them without the reference.

    python tests/golden/gen_golden.py [file.npz ...]

With file names, only those fixtures are written (the others and their
MANIFEST lines are kept as they are).
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
from oracle import ref  # noqa: E402


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


def main(only=()) -> None:
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
    makers = {"quant_ref.npz": lambda: out, "tensor_ref.npz": tensor_cases,
              "bitlinear_ref.npz": bitlinear_cases, "mamba2_ref.npz": mamba2_cases,
              "mamba2_n64_ref.npz": mamba2_n64_cases}
    unknown = set(only) - set(makers)
    if unknown:
        raise SystemExit(f"unknown fixtures: {sorted(unknown)}")
    manifest = os.path.join(HERE, "MANIFEST.sha256")
    digests = {}
    if only and os.path.exists(manifest):
        digests = {name: d for d, name in (l.split() for l in open(manifest) if l.strip())}
    for name, make in makers.items():
        if only and name not in only:
            continue
        path = os.path.join(HERE, name)
        np.savez_compressed(path, **make())
        digests[name] = hashlib.sha256(open(path, "rb").read()).hexdigest()
        print(f"wrote {path} sha256={digests[name]}")
    with open(manifest, "w") as fh:
        fh.writelines(f"{digests[n]}  {n}\n" for n in makers if n in digests)


def _h(rng, shape, scale=1.0, loc=0.0) -> np.ndarray:
    """Seeded normal values rounded to float16 (stored compactly, exact in float32)."""
    return (rng.standard_normal(shape) * scale + loc).astype(np.float16)


def tensor_cases() -> dict:
    rng = np.random.default_rng(20261202)
    out = {}
    # Tensor::rmsnorm rows at the configs' widths and at odd widths (AVX body + tail)
    for k in (768, 1024, 2048, 4096, 1003, 17, 7, 3):
        x = _h(rng, (2, k), scale=float(rng.uniform(0.2, 8.0)))
        out[f"rms_k{k}__x"] = x
        xf = x.astype(np.float32)
        out[f"rms_k{k}__y"] = ref.rmsnorm(xf, 1e-6)
        # RMS_PERI then the AVX2 quantizer: the int8 codes BitLinear::forward multiplies
        codes, scales = oracle.ref_quantize_rows(out[f"rms_k{k}__y"], 8)
        out[f"rms_k{k}__codes"] = np.clip(codes, -127, 127).astype(np.int8)
        out[f"rms_k{k}__scales"] = scales
    # Tensor::softmax rows of config-5-shaped router logits (N(0,1), 8 experts)
    lg = _h(rng, (1024, 8))
    out["softmax__x"] = lg
    out["softmax__y"] = ref.softmax(lg.astype(np.float32))
    lg64 = _h(rng, (64, 64), scale=3.0)
    out["softmax64__x"] = lg64
    out["softmax64__y"] = ref.softmax(lg64.astype(np.float32))
    # elementwise activations over a wide range, both signs
    v = _h(rng, (4096,), scale=6.0)
    g = _h(rng, (4096,), scale=6.0)
    out["act__x"] = v
    out["act__g"] = g
    out["act__silu"] = ref.silu(v.astype(np.float32))
    out["act__silu_gate"] = ref.silu_gate(v.astype(np.float32), g.astype(np.float32))
    out["act__squared_relu"] = ref.squared_relu(v.astype(np.float32))
    # tensor_abs_mean (double sum): sizes on either side of the AVX widths
    for n in (1, 7, 1000, 4099):
        w = _h(rng, (n,), scale=0.05)
        out[f"absmean_n{n}__w"] = w
        out[f"absmean_n{n}__m"] = np.array([ref.abs_mean(w.astype(np.float32))], np.float32)
    # Tensor::rmsnorm_backward with BitLinear's saved x_norm
    for k in (1024, 61):
        x = _h(rng, (4, k), scale=2.0)
        gr = _h(rng, (4, k))
        xf = x.astype(np.float32)
        xn = ref.rmsnorm(xf, 1e-6)
        out[f"rmsbwd_k{k}__x"] = x
        out[f"rmsbwd_k{k}__g"] = gr
        out[f"rmsbwd_k{k}__dx"] = ref.rmsnorm_backward(xf, gr.astype(np.float32), xn, 1e-6)
    return out


def mamba2_cases() -> dict:
    rng = np.random.default_rng(20261204)
    d, H, P, N, G, K = 64, 4, 32, 16, 2, 4
    inner, gs = H * P, G * N
    p = {"w_x": _h(rng, (inner, d), 0.1), "w_z": _h(rng, (inner, d), 0.1),
         "w_B": _h(rng, (gs, d), 0.1), "w_C": _h(rng, (gs, d), 0.1),
         "w_dt": _h(rng, (H, d), 0.1), "dt_bias": _h(rng, (H,), 1.0, -2.0),
         "w_out": _h(rng, (d, inner), 0.1), "conv_w": _h(rng, (inner + 2 * gs, K), 0.5),
         "conv_b": _h(rng, (inner + 2 * gs,), 0.1), "a_log": _h(rng, (H,)),
         "d_skip": _h(rng, (H,)), "norm_w": rng.uniform(0.5, 1.5, inner).astype(np.float16)}
    u = _h(rng, (2, 19, d))
    f32 = {k: v.astype(np.float32) for k, v in p.items()}
    f32.update(H=H, P=P, N=N, G=G)
    out = dict(p)
    out["shape"] = np.array([H, P, N, G], np.int32)
    out["u"] = u
    out["out_packed"] = ref.mamba2_faithful_forward(f32, u.astype(np.float32), packed=True)
    out["out_float"] = ref.mamba2_faithful_forward(f32, u.astype(np.float32), packed=False)
    return out


def mamba2_n64_cases() -> dict:
    """The faithful block at d_state 64 (nsos_config.h's mamba_d_state default), head_dim
    64, two B / C groups, conv 4: two sequences of 41 tokens."""
    rng = np.random.default_rng(20261205)
    d, H, P, N, G, K = 128, 4, 64, 64, 2, 4
    inner, gs = H * P, G * N
    p = {"w_x": _h(rng, (inner, d), 0.1), "w_z": _h(rng, (inner, d), 0.1),
         "w_B": _h(rng, (gs, d), 0.1), "w_C": _h(rng, (gs, d), 0.1),
         "w_dt": _h(rng, (H, d), 0.1), "dt_bias": _h(rng, (H,), 1.0, -2.0),
         "w_out": _h(rng, (d, inner), 0.1), "conv_w": _h(rng, (inner + 2 * gs, K), 0.5),
         "conv_b": _h(rng, (inner + 2 * gs,), 0.1), "a_log": _h(rng, (H,)),
         "d_skip": _h(rng, (H,)), "norm_w": rng.uniform(0.5, 1.5, inner).astype(np.float16)}
    u = _h(rng, (2, 41, d))
    f32 = {k: v.astype(np.float32) for k, v in p.items()}
    f32.update(H=H, P=P, N=N, G=G)
    out = dict(p)
    out["shape"] = np.array([H, P, N, G], np.int32)
    out["u"] = u
    out["out_packed"] = ref.mamba2_faithful_forward(f32, u.astype(np.float32), packed=True)
    return out


def bitlinear_cases() -> dict:
    rng = np.random.default_rng(20261203)
    out = {}
    # (name, M, K, N, exact_linear, magnitude, bias)
    cases = [("rms_mag_bias", 8, 256, 48, False, True, True),
             ("rms_mag", 5, 128, 32, False, True, False),
             ("exact", 6, 192, 40, True, False, False),
             ("exact_bias", 3, 64, 24, True, False, True),
             # more than 16 rows and at most 64 outputs: the float path's skinny MFMA form
             ("gate_rms_mag", 40, 256, 8, False, True, False),
             ("exact_wide_bias", 33, 128, 64, True, False, True)]
    for name, m, k, n, exact, has_mag, has_bias in cases:
        w = _h(rng, (n, k), scale=0.05)
        x = _h(rng, (m, k))
        gr = _h(rng, (m, n))
        mag = rng.uniform(0.5, 1.5, n).astype(np.float16) if has_mag else None
        bias = _h(rng, (n,)) if has_bias else None
        f = lambda a: None if a is None else a.astype(np.float32)
        out[f"{name}__w"] = w
        out[f"{name}__x"] = x
        out[f"{name}__grad"] = gr
        if mag is not None:
            out[f"{name}__mag"] = mag
        if bias is not None:
            out[f"{name}__bias"] = bias
        out[f"{name}__y_packed"] = ref.bitlinear_forward(f(w), f(x), True, exact, f(mag), f(bias))
        out[f"{name}__y_float"] = ref.bitlinear_forward(f(w), f(x), False, exact, f(mag), f(bias))
        bwd = ref.bitlinear_packed_backward(f(w), f(x), f(gr), exact, f(mag), f(bias))
        assert np.array_equal(bwd["y"], out[f"{name}__y_packed"])
        for key in ("dx", "dW", "dmag", "dbias"):
            if key in bwd:
                out[f"{name}__{key}"] = bwd[key]
    return out


if __name__ == "__main__":
    main(tuple(sys.argv[1:]))
