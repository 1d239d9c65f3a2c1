"""Pins the block-norm and decode-conv parts of the CPU oracle (CPU only).

rmsnorm_gated restates RMSNorm(y * SiLU(z)) * gamma (OXN/nsos/src/mamba2.cpp:
2677-2680 over Tensor::silu_gate / rmsnorm / mul); it is checked against the
already-pinned plain rmsnorm (bit for bit when z and gamma are absent), a
float64 evaluation, exact gamma linearity, the z = 0 and constant-row closed
forms.  conv_step restates the decode ring of forward_faithful_step
(src/mamba2.cpp:4072-4090); a chain of steps from an empty ring must equal the
prefill convolution of the same sequence (bit for bit without bias), and the
ring must hold the last W-1 inputs."""
import numpy as np
import pytest


def test_gated_norm_without_gate_is_rmsnorm(orc):
    rng = np.random.default_rng(1)
    y = rng.standard_normal((6, 1027)).astype(np.float32)
    np.testing.assert_array_equal(orc.rmsnorm_gated(y, None, None, eps=1e-6), orc.rmsnorm(y, 1e-6))


def test_gated_norm_matches_float64(orc):
    rng = np.random.default_rng(2)
    y = rng.standard_normal((5, 512)).astype(np.float32)
    z = rng.standard_normal((5, 512)).astype(np.float32)
    gam = rng.uniform(0.5, 1.5, 512).astype(np.float32)
    got = orc.rmsnorm_gated(y, z, gam, eps=1e-5)
    zd = z.astype(np.float64)
    g = y.astype(np.float64) * zd / (1.0 + np.exp(-zd))
    want = g / np.sqrt((g ** 2).mean(axis=1, keepdims=True) + 1e-5) * gam
    np.testing.assert_allclose(got, want, rtol=3e-6, atol=1e-7)


def test_gated_norm_gamma_is_last_multiply(orc):
    rng = np.random.default_rng(3)
    y = rng.standard_normal((3, 64)).astype(np.float32)
    z = rng.standard_normal((3, 64)).astype(np.float32)
    gam = rng.standard_normal(64).astype(np.float32)
    np.testing.assert_array_equal(orc.rmsnorm_gated(y, z, gam),
                                  (orc.rmsnorm_gated(y, z, None) * gam).astype(np.float32))


def test_gated_norm_closed_forms(orc):
    y = np.full((2, 40), 3.0, np.float32)
    # z = 0 closes the gate: g = 0, out = 0
    np.testing.assert_array_equal(orc.rmsnorm_gated(y, np.zeros_like(y)), 0.0)
    # constant row c without a gate: c / sqrt(c^2 + eps)
    out = orc.rmsnorm_gated(y, None, None, eps=1e-5)
    np.testing.assert_allclose(out, 3.0 / np.sqrt(9.0 + 1e-5), rtol=2e-7)


@pytest.mark.parametrize("width", [1, 2, 4])
def test_conv_step_chain_equals_prefill(orc, width):
    rng = np.random.default_rng(width)
    T, C = 9, 12
    x = rng.standard_normal((T, C)).astype(np.float32)
    w = rng.standard_normal((C, width)).astype(np.float32)
    cu = np.array([0, T], np.int32)
    want = orc.conv1d_causal(x, w, cu, bias=None, silu_act=True)
    ring = np.zeros((1, width - 1, C), np.float32) if width > 1 else None
    for t in range(T):
        out, ring = orc.conv_step(x[t:t + 1], w, None, ring, silu_act=True)
        np.testing.assert_array_equal(out[0], want[t])
    if width > 1:
        np.testing.assert_array_equal(ring[0], x[T - (width - 1):])


def test_conv_step_bias_first(orc):
    """The step starts from the bias (the prefill adds it last): equal to rounding."""
    rng = np.random.default_rng(7)
    T, C, W = 6, 8, 4
    x = rng.standard_normal((T, C)).astype(np.float32)
    w = rng.standard_normal((C, W)).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32)
    want = orc.conv1d_causal(x, w, np.array([0, T], np.int32), bias=b, silu_act=False)
    ring = np.zeros((1, W - 1, C), np.float32)
    for t in range(T):
        out, ring = orc.conv_step(x[t:t + 1], w, b, ring, silu_act=False)
        v = np.float32(b)
        for j in range(W):
            src = x[t - (W - 1) + j] if t - (W - 1) + j >= 0 else np.zeros(C, np.float32)
            v = (v.astype(np.float64) + w[:, j].astype(np.float64) * src).astype(np.float32)
        np.testing.assert_allclose(out[0], want[t], rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(out[0], v, rtol=1e-6, atol=1e-6)
