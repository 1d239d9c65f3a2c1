"""JambaBlock composition (Mamba core + MoE feed-forward) on the GPU against the
oracle, stage by stage on the GPU's own upstream tensors (src/jamba.cpp:3158-3375):
core norm and feed-forward norm within the block-norm tolerance (rtol 1e-5 fp32,
2e-2 bf16), the residual adds exact (the RNE bf16 of the fp32 sum), and the MoE
output within the MoE test's bound given the GPU's normalised input."""
import numpy as np
import pytest
import torch

from reimagined_amd import workloads
from reimagined_amd.layers import HybridBlock

pytestmark = pytest.mark.gpu


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("with_gate", [False, True])
def test_hybrid_block_matches_oracle(dev, orc, with_gate):
    rng = np.random.default_rng(21 + int(with_gate))
    params, inp = workloads.config4(seed=13, num_seqs=4, d_model=128, lo=5, hi=90)
    T = int(inp["cu_seqlens"][-1])
    d = params["w_in"].shape[1]
    E, k, f = 4, 2, 256
    w_up = [rng.standard_normal((f, d)).astype(np.float32) for _ in range(E)]
    w_down = [rng.standard_normal((d, f)).astype(np.float32) for _ in range(E)]
    g_core = rng.uniform(0.5, 1.5, d).astype(np.float32)
    g_ff = rng.uniform(0.5, 1.5, d).astype(np.float32)
    gate_w = rng.standard_normal((E, d)).astype(np.float32) if with_gate else None
    blk = HybridBlock(params, w_up, w_down, dev, k=k, core_gamma=g_core, ff_gamma=g_ff,
                      gate_w=gate_w)
    tb = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(dev)
    logits = None if with_gate else torch.from_numpy(
        rng.standard_normal((T, E)).astype(np.float32)).to(dev)
    cu = torch.from_numpy(inp["cu_seqlens"]).to(dev)
    res = blk.forward(tb(inp["x"]), tb(inp["dt"]), tb(inp["B"]), tb(inp["C"]), cu, logits=logits)
    x = _bf(inp["x"])
    core = res["core"].float().cpu().numpy()
    r = res["residual"].float().cpu().numpy()
    out = res["out"].float().cpu().numpy()
    # residual adds: exact bf16 rounding of the fp32 sums
    np.testing.assert_array_equal(r, _bf(x + core))
    np.testing.assert_array_equal(out, _bf(r + res["ff"].float().cpu().numpy()))
    # the core norm fed the Mamba layer: its in_proj input is rmsnorm(x) * gamma
    h_want = orc.rmsnorm_gated(x, None, g_core, eps=1e-6)
    pin, wsi, _ = orc.pack_weights(params["w_in"])
    xz = blk.mamba._buf[T]["xz"].float().cpu().numpy()
    xz_want = orc.bitlinear_forward(_bf(h_want), pin, wsi, xz.shape[1], rms_input=True)
    scale = np.abs(xz_want).max()
    np.testing.assert_allclose(xz, xz_want, rtol=2e-2, atol=2e-2 * scale / 16)
    # feed-forward norm and the MoE on the GPU's residual
    f_want = _bf(orc.rmsnorm_gated(r, None, g_ff, eps=1e-6))
    lg = res["logits"].float().cpu().numpy()
    if with_gate:
        pg, wsg, _ = orc.pack_weights(gate_w)
        lg_want = orc.bitlinear_forward(f_want, pg, wsg, E, rms_input=True)
        np.testing.assert_allclose(lg, lg_want, rtol=2e-2, atol=2e-2 * np.abs(lg_want).max() / 8)
    probs = orc.softmax_rows(lg)
    w, sel = orc.topk_mask(probs, k)
    ff_want = np.zeros((T, d), np.float32)
    for e in range(E):
        pu, wsu, _ = orc.pack_weights(w_up[e])
        pd, wsd, _ = orc.pack_weights(w_down[e])
        hu = orc.squared_relu(orc.bitlinear_forward(f_want, pu, wsu, f, rms_input=True))
        oe = orc.bitlinear_forward(hu, pd, wsd, d, rms_input=True)
        ff_want += w[:, e:e + 1] * oe
    ff = res["ff"].float().cpu().numpy()
    s = np.abs(ff_want).max()
    np.testing.assert_allclose(ff, ff_want, rtol=5e-2, atol=5e-2 * s / 8)
