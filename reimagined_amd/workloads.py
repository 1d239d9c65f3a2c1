"""Seeded synthetic inputs of the five benchmark configurations (numpy, host side).

The distributions follow the configuration text: ternary weights uniform over
{-1, 0, +1} (so the absmean packer returns them unchanged), activations N(0,1),
dt_raw ~ N(-2, 0.5) with delta = softplus(dt_raw) formed in the kernels,
A_log ~ N(0,1) with A = -exp(A_log), B and C ~ N(0, 1/16), D ~ N(0,1),
z ~ N(0,1), ragged lengths uniform in [64, 2048].  numpy's PCG64 generator is
the only source of randomness, so every run and the oracle see the same data.
"""
from __future__ import annotations

import numpy as np


def ternary_uniform(rng: np.random.Generator, n: int, k: int) -> np.ndarray:
    return rng.integers(-1, 2, size=(n, k)).astype(np.float32)


def ragged_lengths(rng: np.random.Generator, count: int, lo: int = 64, hi: int = 2048) -> np.ndarray:
    return rng.integers(lo, hi + 1, size=count).astype(np.int32)


def cu_seqlens(lengths) -> np.ndarray:
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def scan_params(rng: np.random.Generator, T: int, d: int, n: int) -> dict:
    return {
        "x": rng.standard_normal((T, d)).astype(np.float32),
        "dt": rng.normal(-2.0, 0.5, (T, d)).astype(np.float32),
        "a_log": rng.standard_normal((d, n)).astype(np.float32),
        "B": rng.normal(0.0, 0.25, (T, n)).astype(np.float32),
        "C": rng.normal(0.0, 0.25, (T, n)).astype(np.float32),
        "D": rng.standard_normal(d).astype(np.float32),
        "z": rng.standard_normal((T, d)).astype(np.float32),
    }


def config1(seed: int = 1):
    """768x768 ternary BitLinear, 16 tokens of N(0,1) fp32."""
    rng = np.random.default_rng(seed)
    return {"w": ternary_uniform(rng, 768, 768),
            "x": rng.standard_normal((16, 768)).astype(np.float32)}


def config2(seed: int = 2):
    """Selective scan D=768, N=16, batch 1, seq 512, fp32."""
    rng = np.random.default_rng(seed)
    p = scan_params(rng, 512, 768, 16)
    p["cu_seqlens"] = cu_seqlens([512])
    return p


def config3(seed: int = 3, M: int = 4096, K: int = 2048, N: int = 8192):
    """Prefill ternary GEMM M x K x N (activations N(0,1) -> int8 per-token absmax)."""
    rng = np.random.default_rng(seed)
    return {"w": ternary_uniform(rng, N, K),
            "x": rng.standard_normal((M, K)).astype(np.float32)}


def config4(seed: int = 4, num_seqs: int = 32, d_model: int = 1024, expand: int = 2,
            d_state: int = 16, conv: int = 4, lo: int = 64, hi: int = 2048):
    """Hybrid Mamba layer over a packed ragged batch (weights + per-token inputs)."""
    rng = np.random.default_rng(seed)
    d_inner = expand * d_model
    lengths = ragged_lengths(rng, num_seqs, lo, hi)
    cu = cu_seqlens(lengths)
    T = int(cu[-1])
    params = {
        "w_in": ternary_uniform(rng, 2 * d_inner, d_model),
        "w_out": ternary_uniform(rng, d_model, d_inner),
        "conv_w": (rng.standard_normal((d_inner, conv)) * 0.5).astype(np.float32),
        "conv_b": (rng.standard_normal(d_inner) * 0.1).astype(np.float32),
        "a_log": rng.standard_normal((d_inner, d_state)).astype(np.float32),
        "d_skip": rng.standard_normal(d_inner).astype(np.float32),
    }
    inputs = {
        "x": rng.standard_normal((T, d_model)).astype(np.float32),
        "dt": rng.normal(-2.0, 0.5, (T, d_inner)).astype(np.float32),
        "B": rng.normal(0.0, 0.25, (T, d_state)).astype(np.float32),
        "C": rng.normal(0.0, 0.25, (T, d_state)).astype(np.float32),
        "cu_seqlens": cu,
    }
    return params, inputs


def config5(seed: int = 5, rows: int = 8192, experts: int = 8, d_model: int = 1024,
            d_ff: int = 4096, decode_rows: int = 256, d_inner: int = 2048, d_state: int = 16):
    """Ternary MoE FFN (top-2) + one Mamba decode step over decode_rows sequences."""
    rng = np.random.default_rng(seed)
    moe = {
        "w_up": [ternary_uniform(rng, d_ff, d_model) for _ in range(experts)],
        "w_down": [ternary_uniform(rng, d_model, d_ff) for _ in range(experts)],
        "x": rng.standard_normal((rows, d_model)).astype(np.float32),
        "logits": rng.standard_normal((rows, experts)).astype(np.float32),
    }
    dec = scan_params(rng, decode_rows, d_inner, d_state)
    dec["state"] = rng.normal(0.0, 0.1, (decode_rows, d_inner, d_state)).astype(np.float32)
    return moe, dec
