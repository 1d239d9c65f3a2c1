"""JambaBlock composition (Mamba core + MoE feed-forward) on the GPU against the
oracle, stage by stage on the GPU's own upstream tensors (src/jamba.cpp:3158-3375):

  * the core and feed-forward norms within the block-norm tolerance (the GPU sums
    squares in a wave tree, the reference in order: rtol 1e-5 in fp32, one bf16 ulp
    after rounding);
  * the in_proj on the GPU's normed input bit-exact (bf16 = RNE of the oracle's fp32);
  * the router gate, by default the reference's float path (MoERouter marks the gate
    quantization-sensitive, src/jamba.cpp:8086-8098): rmsnorm(f) @ W^T * magnitude
    within the fp32 bound 1e-4 / 1e-5; with ternary_gate the ternary BitLinear
    bit-exact;
  * the MoE feed-forward on the GPU's f and logits within the bf16 bound 2e-2;
  * the residual adds exact (the RNE bf16 of the fp32 sums)."""
import numpy as np
import pytest
import torch

from reimagined_amd import workloads
from reimagined_amd.layers import HybridBlock

pytestmark = pytest.mark.gpu


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).float().numpy()


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("gate", ["logits", "float", "ternary"])
def test_hybrid_block_matches_oracle(dev, orc, gate):
    rng = np.random.default_rng(21 + len(gate))
    params, inp = workloads.config4(seed=13, num_seqs=4, d_model=128, lo=5, hi=90)
    T = int(inp["cu_seqlens"][-1])
    d = params["w_in"].shape[1]
    E, k, f = 4, 2, 256
    w_up = [rng.standard_normal((f, d)).astype(np.float32) for _ in range(E)]
    w_down = [rng.standard_normal((d, f)).astype(np.float32) for _ in range(E)]
    g_core = rng.uniform(0.5, 1.5, d).astype(np.float32)
    g_ff = rng.uniform(0.5, 1.5, d).astype(np.float32)
    gate_w = (rng.standard_normal((E, d)) / np.sqrt(d)).astype(np.float32)
    gate_mag = rng.uniform(0.5, 1.5, E).astype(np.float32)
    kw = {} if gate == "logits" else dict(gate_w=gate_w, gate_magnitude=gate_mag,
                                         ternary_gate=gate == "ternary")
    blk = HybridBlock(params, w_up, w_down, dev, k=k, core_gamma=g_core, ff_gamma=g_ff, **kw)
    tb = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(dev)
    logits = None if gate != "logits" else torch.from_numpy(
        rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    cu = torch.from_numpy(inp["cu_seqlens"]).to(dev)
    res = blk.forward(tb(inp["x"]), tb(inp["dt"]), tb(inp["B"]), tb(inp["C"]), cu, logits=logits)
    x = _bf(inp["x"])
    core, r, out, h, fin = (_np(res[key]) for key in ("core", "residual", "out", "h", "f"))
    # residual adds: exact bf16 rounding of the fp32 sums
    np.testing.assert_array_equal(r, _bf(x + core))
    np.testing.assert_array_equal(out, _bf(r + _np(res["ff"])))
    # block norms: within one bf16 ulp of the oracle's in-order norm
    np.testing.assert_allclose(h, _bf(orc.rmsnorm_gated(x, None, g_core, eps=1e-6)),
                               rtol=8e-3, atol=1e-6)
    np.testing.assert_allclose(fin, _bf(orc.rmsnorm_gated(r, None, g_ff, eps=1e-6)),
                               rtol=8e-3, atol=1e-6)
    # in_proj on the GPU's normed input: bit-exact
    pin, wsi, _ = orc.pack_weights(params["w_in"])
    xz = _np(blk.mamba._buf[T]["xz"])
    np.testing.assert_array_equal(xz, _bf(orc.bitlinear_forward(h, pin, wsi, xz.shape[1],
                                                                 rms_input=True)))
    # router gate over the GPU's f
    lg = _np(res["logits"])
    if gate == "float":
        want = orc.linear_f32(fin, gate_w, True, gate_mag)
        np.testing.assert_allclose(lg, want, rtol=1e-4, atol=1e-5 * np.abs(want).max())
    elif gate == "ternary":
        pg, wsg, _ = orc.pack_weights(gate_w)
        np.testing.assert_array_equal(lg, orc.bitlinear_forward(fin, pg, wsg, E, 8, True,
                                                                gate_mag))
    # MoE feed-forward on the GPU's f and logits
    probs = orc.softmax_rows(lg)
    w, sel = orc.topk_mask(probs, k)
    ff_want = np.zeros((T, d), np.float32)
    for e in range(E):
        pu, wsu, _ = orc.pack_weights(w_up[e])
        pd, wsd, _ = orc.pack_weights(w_down[e])
        hu = orc.squared_relu(orc.bitlinear_forward(fin, pu, wsu, f, rms_input=True))
        oe = orc.bitlinear_forward(hu, pd, wsd, d, rms_input=True)
        ff_want += w[:, e:e + 1] * oe
    np.testing.assert_allclose(_np(res["ff"]), ff_want, rtol=2e-2,
                               atol=2e-2 * np.abs(ff_want).max() / 64)
