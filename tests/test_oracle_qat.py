"""Pins of the oracle's QAT fake-quant restatement (OXN/nsos/src/bitnet_gpu_dispatch.cpp:193-325)
by constructed cases with closed-form answers, invariants of the quantizers, and agreement with
the oracle's independent BitLinear packing path (src/bitlinear.cpp:174, 1359-1379)."""
import numpy as np

from oracle import oracle as orc


def test_ternary_thresholds_at_unit_scale():
    # scale 1: 1 + 1e-8f rounds to 1, so v = w and the cut points are exactly +-0.5 (exclusive)
    w = np.array([0.5, np.nextafter(np.float32(0.5), np.float32(1)), -0.5,
                  np.nextafter(np.float32(-0.5), np.float32(-1)), 0.0, 2.0, -3.0], np.float32)
    np.testing.assert_array_equal(orc.qat_fake_quant_ternary(w, 1.0),
                                  np.array([0, 1, 0, -1, 0, 1, -1], np.float32))


def test_ternary_outputs_are_scaled_codes_and_idempotent():
    rng = np.random.default_rng(0)
    w = rng.standard_normal(4096).astype(np.float32)
    out, scale = orc.qat_fake_quant_ternary_absmean(w)
    assert set(np.unique(out)) <= {-scale, np.float32(0), scale}
    np.testing.assert_array_equal(orc.qat_fake_quant_ternary(out, scale), out)


def test_absmean_scale_matches_packing_path():
    w = np.array([1, -1, 2, -2], np.float32)
    _, scale = orc.qat_fake_quant_ternary_absmean(w)
    assert scale == np.float32(1.5)
    rng = np.random.default_rng(1)
    w = rng.standard_normal((64, 96)).astype(np.float32)
    out, scale = orc.qat_fake_quant_ternary_absmean(w)
    assert scale == np.float32(orc.weight_scale(w))
    # away from the cut points the codes equal the packing path's (which divides instead of
    # multiplying by the reciprocal)
    _, _, codes = orc.pack_weights(w)
    v = np.abs(w / np.float32(scale + np.float32(1e-8)))
    far = np.abs(v - 0.5) > 1e-5
    np.testing.assert_array_equal((out / scale)[far], codes.reshape(w.shape)[far].astype(np.float32))


def test_activation_ties_round_half_away():
    # bits 2: q_max 1; row max 2 -> scale 0.5, the second element lands on 0.5 exactly
    out = orc.qat_fake_quant_activations(np.array([[2.0, 1.0, -1.0, 0.0]], np.float32), 2)
    np.testing.assert_array_equal(out, np.array([[2.0, 2.0, -2.0, 0.0]], np.float32))


def test_activation_grid_and_error_bound():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((7, 333)).astype(np.float32)
    for bits in (2, 4, 8):
        out = orc.qat_fake_quant_activations(x, bits)
        q_max = 1.0 if bits <= 2 else 2 ** (bits - 1) - 1
        denom = np.abs(x).max(axis=1, keepdims=True) + 1e-8
        step = denom / q_max
        k = out / step
        np.testing.assert_allclose(k, np.round(k), atol=1e-3)     # on the code grid
        assert np.all(np.abs(np.round(k)) <= q_max)
        assert np.all(np.abs(out - x) <= step / 2 * (1 + 1e-5) + 1e-7)  # rounding error bound
        np.testing.assert_allclose(np.abs(out).max(axis=1), denom[:, 0], rtol=1e-6)


def test_ste_clip_zeroes_only_saturated_weights():
    w = np.array([1.0, np.nextafter(np.float32(1), np.float32(2)), -2.0, 0.5, -1.0], np.float32)
    dw = np.arange(1, 6, dtype=np.float32)
    np.testing.assert_array_equal(orc.qat_ste_clip(dw, w, 1.0),
                                  np.array([1, 0, 0, 4, 5], np.float32))
