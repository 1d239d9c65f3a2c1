"""The float (quantization-sensitive) BitLinear path and the packed STE backward on the GPU.

Against the oracle (double-accumulated restatement) and against the reference
build's own outputs (tests/golden/bitlinear_ref.npz): fp32 outputs within
1e-4 relative / 1e-5 absolute of the output scale (the north-star fp32 bound;
both sides sum in their own order), bf16 outputs within 2e-2 relative; the
normalised input of RMS_PERI is the bit-exact x * inv of the quantizer path."""
import os

import numpy as np
import pytest
import torch

from reimagined_amd import ops

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "bitlinear_ref.npz")


def _close(got, want, rtol=1e-4, atol=1e-5, what=""):
    scale = max(float(np.abs(want).max()), 1e-30)
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol * scale, err_msg=what)


@pytest.mark.parametrize("m,k,n", [(40, 1024, 160), (40796 // 64, 1024, 160), (5, 1024, 160),
                                   (1, 1024, 160), (300, 1024, 8), (8192 // 8, 1024, 8),
                                   (1, 64, 3), (129, 256, 130), (17, 4096, 17), (16, 64, 16),
                                   (40796 // 16, 1024, 64), (100, 1000, 33), (33, 72, 48),
                                   (4097, 512, 64), (257, 1028, 17), (18, 4, 1)])
@pytest.mark.parametrize("rms", [False, True])
def test_linear_f32_matches_oracle(dev, orc, m, k, n, rms):
    rng = np.random.default_rng(m * 31 + n)
    x = (rng.standard_normal((m, k)) * rng.uniform(0.5, 4.0)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    mag = rng.uniform(0.5, 1.5, n).astype(np.float32)
    bias = rng.standard_normal(n).astype(np.float32)
    t = lambda a: torch.from_numpy(a).to(dev)
    for mg, b in ((None, None), (mag, bias), (None, bias)):
        y = ops.linear_f32(t(x), t(w), rms, None if mg is None else t(mg),
                           None if b is None else t(b))
        want = orc.linear_f32(x, w, rms, mg, b)
        _close(y.cpu().numpy(), want, what=f"mag={mg is not None} bias={b is not None}")


@pytest.mark.parametrize("m,n,k", [(600, 160, 1024), (3, 160, 1024), (700, 8, 1024),
                                   (700, 64, 1024), (70, 40, 1028), (65, 33, 72)])
def test_linear_f32_bf16_io(dev, orc, m, n, k):
    rng = np.random.default_rng(m + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) / np.sqrt(k)).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    y = ops.linear_f32(xb.to(dev), torch.from_numpy(w).to(dev), True, out_dtype=torch.bfloat16)
    want = orc.linear_f32(xb.float().numpy(), w, True)
    _close(y.float().cpu().numpy(), want, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("name", ["rms_mag_bias", "rms_mag", "exact", "exact_bias", "gate_rms_mag",
                                  "exact_wide_bias"])
def test_linear_f32_matches_reference_golden(dev, name):
    g = np.load(GOLDEN, allow_pickle=False)
    f = lambda key: (torch.from_numpy(g[f"{name}__{key}"].astype(np.float32)).to(dev)
                     if f"{name}__{key}" in g.files else None)
    exact = name.startswith("exact")
    y = ops.linear_f32(f("x"), f("w"), not exact, None if exact else f("mag"), f("bias"))
    _close(y.cpu().numpy(), g[f"{name}__y_float"], rtol=1e-5, atol=1e-6)


def _ste_case(orc, dev, x, w, grad, rms, mag, use_bias):
    o = orc.bitlinear_ste_backward(x, w, grad, rms, mag, use_bias)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    got = ops.bitlinear_ste_backward(t(x), t(o["q"]), t(o["act_scale"]), t(w),
                                     t(o["packed"].view(np.int32)), o["weight_scale"], t(grad),
                                     rms, None if mag is None else t(mag), use_bias)
    return o, {k: v.cpu().numpy() for k, v in got.items()}


@pytest.mark.parametrize("m,k,n", [(8, 256, 48), (300, 1024, 256), (1000, 512, 700),
                                   (33, 2048, 1024), (1, 16, 4), (257, 128, 132)])
@pytest.mark.parametrize("rms,with_mag,use_bias", [(True, True, True), (False, False, False),
                                                   (False, False, True), (True, True, False)])
def test_ste_backward_matches_oracle(dev, orc, m, k, n, rms, with_mag, use_bias):
    rng = np.random.default_rng(m + 7 * k + n)
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    grad = rng.standard_normal((m, n)).astype(np.float32)
    mag = rng.uniform(0.5, 1.5, n).astype(np.float32) if with_mag else None
    o, got = _ste_case(orc, dev, x, w, grad, rms, mag, use_bias)
    for key in ("dx", "dW", "dmag", "dbias"):
        if key in o:
            assert key in got
            _close(got[key], o[key], what=key)
    # the clip zeroes exactly the entries the oracle zeroes
    clip = np.abs(w / np.float32(o["weight_scale"] + np.float32(1e-8))) > 1.0
    assert np.all(got["dW"][clip] == 0.0)


@pytest.mark.parametrize("name", ["rms_mag_bias", "rms_mag", "exact", "exact_bias", "gate_rms_mag",
                                  "exact_wide_bias"])
def test_ste_backward_matches_reference_golden(dev, orc, name):
    g = np.load(GOLDEN, allow_pickle=False)
    f = lambda key: g[f"{name}__{key}"].astype(np.float32) if f"{name}__{key}" in g.files else None
    exact = name.startswith("exact")
    o, got = _ste_case(orc, dev, f("x"), f("w"), f("grad"), not exact, f("mag"),
                       f("bias") is not None)
    for key in ("dx", "dW", "dmag", "dbias"):
        if f"{name}__{key}" in g.files:
            _close(got[key], g[f"{name}__{key}"], rtol=1e-5, atol=1e-6, what=key)
