"""QAT fake-quant kernels on the GPU against the CPU oracle (src/bitnet_gpu_dispatch.cpp:193-325):
every output bit-exact, the device absmean scale equal to the CPU's double-sum scale."""
import numpy as np
import pytest
import torch

from reimagined_amd import ops

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [1, 255, 4096, 1 << 20, 3_000_001])
def test_fake_quant_ternary_absmean_bit_exact(dev, orc, n):
    rng = np.random.default_rng(n)
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    want, want_scale = orc.qat_fake_quant_ternary_absmean(w)
    out, scale = ops.qat_fake_quant_ternary_absmean(torch.from_numpy(w).to(dev))
    assert scale.item() == want_scale
    np.testing.assert_array_equal(out.cpu().numpy(), want)


def test_fake_quant_ternary_given_scale_thresholds(dev, orc):
    w = np.array([0.5, np.nextafter(np.float32(0.5), np.float32(1)), -0.5, -0.5000001, 0, 7,
                  -7, 0.1], np.float32)
    for scale in (1.0, 0.25, 0.0371):
        want = orc.qat_fake_quant_ternary(w * scale, scale)
        got = ops.qat_fake_quant_ternary(torch.from_numpy(w * np.float32(scale)).to(dev), scale)
        np.testing.assert_array_equal(got.cpu().numpy(), want)
    with pytest.raises(ValueError, match="finite positive scale"):
        ops.qat_fake_quant_ternary(torch.zeros(4, device=dev), 0.0)


@pytest.mark.parametrize("shape,bits", [((1, 7), 8), ((33, 1024), 8), ((5, 3000), 4),
                                        ((64, 96), 2), ((3, 257), 3)])
def test_fake_quant_activations_bit_exact(dev, orc, shape, bits):
    rng = np.random.default_rng(shape[0] * 7 + bits)
    x = rng.standard_normal(shape).astype(np.float32)
    x[0, 0] = 2.0
    x[0, -1] = 1.0  # bits 2: lands on a .5 tie (half away from zero)
    want = orc.qat_fake_quant_activations(x, bits)
    got = ops.qat_fake_quant_activations(torch.from_numpy(x).to(dev), bits)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    with pytest.raises(ValueError, match="precision_bits"):
        ops.qat_fake_quant_activations(torch.from_numpy(x).to(dev), 9)


def test_ste_clip_host_and_device_scale(dev, orc):
    rng = np.random.default_rng(5)
    w = (rng.standard_normal((128, 300)) * 0.05).astype(np.float32)
    dw = rng.standard_normal(w.shape).astype(np.float32)
    _, scale = orc.qat_fake_quant_ternary_absmean(w)
    want = orc.qat_ste_clip(dw, w, scale)
    assert 0 < np.sum(want == 0) < w.size  # some weights saturate, most do not
    wd = torch.from_numpy(w).to(dev)
    got = ops.qat_ste_clip_weight_grad(torch.from_numpy(dw).to(dev), wd, float(scale))
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    _, sdev = ops.qat_fake_quant_ternary_absmean(wd)
    got = ops.qat_ste_clip_weight_grad(torch.from_numpy(dw).to(dev), wd, sdev)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
