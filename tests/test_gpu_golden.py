"""The GPU path against the reference build's own outputs (tests/golden/, written by
tests/golden/gen_golden.py from oracle/_ref): the RMS_PERI int8 codes and act_scale
bit for bit, the BitLinear packed forward (magnitude and bias included) bit for bit,
and the router's probabilities within 1e-6 with the selections equal to the top-k of
the reference's probabilities."""
import os

import numpy as np
import pytest
import torch

from reimagined_amd import ops

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _g(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


@pytest.mark.parametrize("k", [768, 1024, 2048, 4096, 1003, 17, 7, 3])
def test_rms_peri_codes_match_reference(dev, k):
    g = _g("tensor_ref.npz")
    x = torch.from_numpy(g[f"rms_k{k}__x"].astype(np.float32)).to(dev)
    q, s = ops.quantize_activations_bitnet(x, 8, rms_input=True)
    np.testing.assert_array_equal(q.cpu().numpy(), g[f"rms_k{k}__codes"])
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32),
                                  g[f"rms_k{k}__scales"].view(np.uint32))


@pytest.mark.parametrize("name", ["rms_mag_bias", "rms_mag", "exact", "exact_bias", "gate_rms_mag",
                                  "exact_wide_bias"])
def test_bitlinear_packed_forward_matches_reference(dev, orc, name):
    g = _g("bitlinear_ref.npz")
    f = lambda key: (torch.from_numpy(g[f"{name}__{key}"].astype(np.float32)).to(dev)
                     if f"{name}__{key}" in g.files else None)
    w = g[f"{name}__w"].astype(np.float32)
    x = f("x")
    packed, ws, _ = orc.pack_weights(w)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    m, k = x.shape
    y = ops.bitnet_gemm_158bit_gpu(x, pk, ws, m, k, w.shape[0], 8, f("mag"), f("bias"),
                                   rms_input=not name.startswith("exact"))
    want = g[f"{name}__y_packed"]
    np.testing.assert_array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name,k", [("softmax", 2), ("softmax", 1), ("softmax64", 8),
                                    ("softmax", 8)])
def test_route_matches_reference_softmax(dev, orc, name, k):
    g = _g("tensor_ref.npz")
    logits = g[f"{name}__x"].astype(np.float32)
    probs = g[f"{name}__y"]
    r = ops.moe_route(torch.from_numpy(logits).to(dev), k)
    want_w, want_sel = orc.topk_mask(probs, k)
    np.testing.assert_array_equal(r["selected"].cpu().numpy(), want_sel)
    np.testing.assert_allclose(r["weights"].cpu().numpy(), want_w, rtol=1e-6, atol=1e-7)
    if k == logits.shape[1]:   # k == E: the raw softmax, not renormalised
        np.testing.assert_allclose(r["weights"].cpu().numpy(), probs, rtol=1e-6, atol=1e-7)
