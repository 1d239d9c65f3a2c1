"""Block norms and the decode conv ring on the GPU against the CPU oracle.

Tolerances (fp32 I/O): the row sum of squares is a wave tree on the GPU and an
index-order sum in the oracle, so norms agree to a few ulp of the sum:
rtol 1e-5, atol 1e-6 (inside the north-star 1e-4 / 1e-5).  bf16 I/O: the oracle
runs in fp32 on the bf16-rounded inputs; outputs within 2e-2 relative.  The
residual add is exact (fp32) or exactly the round-to-nearest-even bf16 of the
fp32 sum."""
import numpy as np
import pytest
import torch

from reimagined_amd import ops

pytestmark = pytest.mark.gpu


def _t(dev, a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(dev)


def _bf(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).float().numpy()


@pytest.mark.parametrize("rows,dim", [(7, 2048), (5, 37), (1, 1), (130, 768)])
@pytest.mark.parametrize("gated,gamma", [(True, True), (True, False), (False, True), (False, False)])
def test_rmsnorm_gated_matches_oracle(dev, orc, rows, dim, gated, gamma):
    rng = np.random.default_rng(rows * 7 + dim)
    y = rng.standard_normal((rows, dim)).astype(np.float32)
    z = rng.standard_normal((rows, dim)).astype(np.float32) if gated else None
    g = rng.uniform(0.5, 1.5, dim).astype(np.float32) if gamma else None
    got = ops.rmsnorm_gated(_t(dev, y), None if z is None else _t(dev, z),
                            None if g is None else _t(dev, g), eps=1e-5)
    want = orc.rmsnorm_gated(y, z, g, eps=1e-5)
    np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-5, atol=1e-6)


def test_rmsnorm_gated_bf16(dev, orc):
    rng = np.random.default_rng(11)
    y = rng.standard_normal((33, 2048)).astype(np.float32)
    z = rng.standard_normal((33, 2048)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 2048).astype(np.float32)
    got = ops.rmsnorm_gated(_t(dev, y, torch.bfloat16), _t(dev, z, torch.bfloat16), _t(dev, g))
    want = orc.rmsnorm_gated(_bf(y), _bf(z), g)
    np.testing.assert_allclose(got.float().cpu().numpy(), want, rtol=2e-2, atol=2e-2)
    got32 = ops.rmsnorm_gated(_t(dev, y, torch.bfloat16), _t(dev, z, torch.bfloat16), _t(dev, g),
                              out_dtype=torch.float32)
    np.testing.assert_allclose(got32.cpu().numpy(), want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_add_rmsnorm(dev, orc, dtype):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((19, 1024)).astype(np.float32)
    d = rng.standard_normal((19, 1024)).astype(np.float32)
    g = rng.uniform(0.5, 1.5, 1024).astype(np.float32)
    res, norm = ops.add_rmsnorm(_t(dev, x, dtype), _t(dev, d, dtype), _t(dev, g), eps=1e-6)
    if dtype == torch.float32:
        want_res = x + d
        np.testing.assert_array_equal(res.cpu().numpy(), want_res)
        np.testing.assert_allclose(norm.cpu().numpy(), orc.rmsnorm_gated(want_res, None, g, 1e-6),
                                   rtol=1e-5, atol=1e-6)
    else:
        want_res = _bf(_bf(x) + _bf(d))
        np.testing.assert_array_equal(res.float().cpu().numpy(), want_res)
        np.testing.assert_allclose(norm.float().cpu().numpy(),
                                   orc.rmsnorm_gated(want_res, None, g, 1e-6), rtol=2e-2, atol=2e-2)
    res2, none = ops.add_rmsnorm(_t(dev, x, dtype), _t(dev, d, dtype), want_norm=False)
    assert none is None
    np.testing.assert_array_equal(res2.float().cpu().numpy(), res.float().cpu().numpy())


@pytest.mark.parametrize("width,bias,dtype", [(4, True, torch.float32), (1, False, torch.float32),
                                              (2, True, torch.float32), (4, True, torch.bfloat16)])
def test_conv_step_chain_matches_oracle(dev, orc, width, bias, dtype):
    rng = np.random.default_rng(width * 3 + int(bias))
    R, C, T = 5, 300, 7
    xs = rng.standard_normal((T, R, C)).astype(np.float32)
    if dtype == torch.bfloat16:
        xs = _bf(xs)
    w = rng.standard_normal((C, width)).astype(np.float32)
    b = rng.standard_normal(C).astype(np.float32) if bias else None
    ring_np = (rng.standard_normal((R, width - 1, C)) * 0.5).astype(np.float32) if width > 1 else None
    ring = _t(dev, ring_np) if width > 1 else None
    wt, bt = _t(dev, w), (None if b is None else _t(dev, b))
    for t in range(T):
        out = ops.conv_step(_t(dev, xs[t], dtype), wt, bt, ring, out_dtype=torch.float32)
        want, ring_np = orc.conv_step(xs[t], w, b, ring_np, silu_act=True)
        np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-6)
    if width > 1:
        np.testing.assert_array_equal(ring.cpu().numpy(), ring_np)


def test_conv_step_strided_input_and_rejections(dev, orc):
    rng = np.random.default_rng(9)
    R, C, W = 3, 64, 4
    wide = rng.standard_normal((R, 3 * C)).astype(np.float32)
    w = rng.standard_normal((C, W)).astype(np.float32)
    ring = torch.zeros((R, W - 1, C), device=dev)
    xt = _t(dev, wide)[:, C:2 * C]
    out = ops.conv_step(xt, _t(dev, w), None, ring, apply_silu=False)
    want, _ = orc.conv_step(wide[:, C:2 * C], w, None, np.zeros((R, W - 1, C), np.float32),
                            silu_act=False)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-6, atol=1e-6)
    with pytest.raises(ValueError):
        ops.conv_step(xt, _t(dev, w), None, torch.zeros((R, W, C), device=dev))
    with pytest.raises(ValueError):
        ops.rmsnorm_gated(_t(dev, wide), gamma=torch.ones(5, device=dev))


@pytest.mark.parametrize("rows,dim,dtype,keep", [(40, 2048, torch.float32, False),
                                                 (37, 2048, torch.float32, True),
                                                 (9, 1024, torch.bfloat16, False),
                                                 (5, 4096, torch.bfloat16, True),
                                                 (6, 120, torch.float32, False)])
def test_rmsnorm_gated_quant_equals_two_passes(dev, orc, rows, dim, dtype, keep):
    """The gated norm with out_proj's int8 input quantization in one pass equals the
    gated norm followed by quantize_act_i8 on its stored rows, bit for bit (dim 120
    takes the two passes themselves); the codes also match the oracle's quantization of
    the GPU's normed rows."""
    rng = np.random.default_rng(rows + dim)
    y = _t(dev, rng.standard_normal((rows, dim)), dtype)
    z = _t(dev, rng.standard_normal((rows, dim)), dtype)
    g = _t(dev, rng.uniform(0.5, 1.5, dim))
    q, s, out = ops.rmsnorm_gated_quant(y, z, g, eps=1e-5, want_out=keep)
    normed = ops.rmsnorm_gated(y, z, g, eps=1e-5)
    q2, s2 = ops.quantize_activations_bitnet(normed, 8)
    np.testing.assert_array_equal(q.cpu().numpy(), q2.cpu().numpy())
    np.testing.assert_array_equal(s.cpu().numpy(), s2.cpu().numpy())
    if keep:
        np.testing.assert_array_equal(out.float().cpu().numpy(), normed.float().cpu().numpy())
    wq, ws = orc.quantize_act(normed.float().cpu().numpy(), 8)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)
