"""Faithful Mamba-2 block (Mamba2SSD::forward_faithful and its decode step) on the GPU
against the oracle's composition, stage by stage on the GPU's own upstream tensors
(src/mamba2.cpp:2360-2681), with the reference's mixed precision (584-662):

  * x and z: ternary BitLinear in exact-linear mode (no input norm, no magnitude),
    bit-exact;
  * B, C, dt: the float path (quantization-sensitive), dt with its bias, within the
    fp32 bound 1e-4 / 1e-5 of the output scale;
  * conv / scan / gated norm within the fp32 bounds of their own tests (1e-4 rel,
    1e-5 abs; norm 1e-5 / 1e-6); out_proj (exact-linear ternary, src/mamba2.cpp:514)
    bit-exact;
  * the whole block against a reference build's Mamba2SSD::forward (golden).

The decode step equals the prefill token by token (to the conv's bias-first rounding
and int8 code flips: 1e-3 of the output scale), and a HIP-graph replay of the step
equals the eager step bit for bit on every replay.  Its fused launch (conv ring, state
step, gated norm, out_proj quantization) equals the chain of the separate GPU ops
(conv_step x3, selective_scan_step, rmsnorm_gated, quantize_act_i8) bit for bit where
the gated norm's register path sums in the same order, and the oracle's decode chain
within the fp32 bounds."""
import numpy as np
import pytest
import torch

from reimagined_amd.layers import Mamba2Block

pytestmark = pytest.mark.gpu


def _params(rng, d=64, H=4, P=16, N=16, G=2, K=4):
    inner, gs = H * P, G * N
    w = lambda n, k: rng.standard_normal((n, k)).astype(np.float32)
    return {
        "w_x": w(inner, d), "w_z": w(inner, d), "w_B": w(gs, d) / 8, "w_C": w(gs, d) / 8,
        "w_dt": w(H, d) / 8, "w_out": w(d, inner),
        "dt_bias": (rng.standard_normal(H) - 2.0).astype(np.float32),
        "conv_w": (rng.standard_normal((inner + 2 * gs, K)) * 0.5).astype(np.float32),
        "conv_b": (rng.standard_normal(inner + 2 * gs) * 0.1).astype(np.float32),
        "a_log": rng.standard_normal(H).astype(np.float32),
        "d_skip": rng.standard_normal(H).astype(np.float32),
        "norm_w": rng.uniform(0.5, 1.5, inner).astype(np.float32),
        "H": H, "P": P, "N": N, "G": G,
    }


def _np(t):
    return t.float().cpu().numpy()


@pytest.mark.parametrize("P,N,chunk", [(16, 16, -1), (64, 64, 0), (64, 64, 8), (64, 32, 4)])
def test_mamba2_block_prefill_matches_oracle(dev, orc, P, N, chunk):
    """Stage by stage against the oracle, at d_state 16 (the quad scan) and at 32 / 64 (the
    LDS-staged scan, sequential and time-chunked)."""
    rng = np.random.default_rng(3 + N + P + chunk)
    p = _params(rng, P=P, N=N)
    H, P, N, G = p["H"], p["P"], p["N"], p["G"]
    inner, gs = H * P, G * N
    blk = Mamba2Block(p, dev)
    lengths = [5, 17, 1, 30]
    cu = np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)
    T = int(cu[-1])
    u = rng.standard_normal((T, 64)).astype(np.float32)
    res = blk.forward(torch.from_numpy(u).to(dev), torch.from_numpy(cu).to(dev), keep_normed=True,
                      chunk_tokens=chunk)
    # x, z: ternary exact-linear (no RMS_PERI, no magnitude), bit-exact
    for key, wk in (("x", "w_x"), ("z", "w_z")):
        pk, ws, _ = orc.pack_weights(p[wk])
        want = orc.bitlinear_forward(u, pk, ws, p[wk].shape[0], rms_input=False)
        np.testing.assert_array_equal(_np(res[key]), want)
    # B, C, dt: float linears of u, dt plus its bias (within the fp32 bound)
    Bv = orc.linear_f32(u, p["w_B"])
    Cv = orc.linear_f32(u, p["w_C"])
    dtv = orc.linear_f32(u, p["w_dt"], bias=p["dt_bias"])
    for got, want in ((res["Bv"], Bv), (res["Cv"], Cv), (res["dt"], dtv)):
        np.testing.assert_allclose(_np(got), want, rtol=1e-4, atol=1e-5 * np.abs(want).max())
    Bv, Cv = _np(res["Bv"]), _np(res["Cv"])
    # conv + SiLU on B and C
    cw, cb = p["conv_w"], p["conv_b"]
    Bc = orc.conv1d_causal(Bv, cw[inner:inner + gs], cu, bias=cb[inner:inner + gs], silu_act=True)
    Cc = orc.conv1d_causal(Cv, cw[inner + gs:], cu, bias=cb[inner + gs:], silu_act=True)
    np.testing.assert_allclose(_np(res["B"]), Bc, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(res["C"]), Cc, rtol=1e-5, atol=1e-6)
    # conv on x fused into the per-head scan (no gate inside the scan)
    xc = orc.conv1d_causal(_np(res["x"]), cw[:inner], cu, bias=cb[:inner], silu_act=True)
    y, fin = orc.selective_scan(xc, _np(res["dt"]), p["a_log"], _np(res["B"]), _np(res["C"]),
                                p["d_skip"], None, cu, H, P, N, G, gate_silu=False)
    np.testing.assert_allclose(_np(res["y"]), y, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(_np(res["final_state"]), fin, rtol=1e-4, atol=1e-5)
    # gated RMSNorm epilogue and out_proj
    normed = orc.rmsnorm_gated(_np(res["y"]), _np(res["z"]), p["norm_w"], eps=1e-5)
    np.testing.assert_allclose(_np(res["normed"]), normed, rtol=1e-5, atol=1e-6)
    pk, ws, _ = orc.pack_weights(p["w_out"])
    out = orc.bitlinear_forward(_np(res["normed"]), pk, ws, 64, rms_input=False)
    np.testing.assert_array_equal(_np(res["out"]), out)


@pytest.mark.parametrize("R", [3, 1])
def test_mamba2_decode_step_equals_prefill(dev, orc, R):
    """(one row: the projections in one grouped launch and the out_proj GEMV with the
    norm prologue; three rows: the separate launches)"""
    rng = np.random.default_rng(5)
    p = _params(rng, H=2, P=32, G=1)
    blk = Mamba2Block(p, dev)
    T = 7
    u = rng.standard_normal((R, T, 64)).astype(np.float32)
    cu = torch.arange(R + 1, dtype=torch.int32, device=dev) * T
    pre = blk.forward(torch.from_numpy(u.reshape(R * T, 64)).to(dev), cu)["out"]
    pre = _np(pre).reshape(R, T, 64)
    dec = blk.new_decode_state(R, dev)
    for t in range(T):
        out = _np(blk.step(torch.from_numpy(np.ascontiguousarray(u[:, t])).to(dev), dec))
        scale = np.abs(pre[:, t]).max()
        np.testing.assert_allclose(out, pre[:, t], rtol=1e-3, atol=1e-3 * scale)


@pytest.mark.parametrize("R", [4, 1])
def test_mamba2_step_graph_replay_equals_eager(dev, orc, R):
    rng = np.random.default_rng(8)
    p = _params(rng)
    blk = Mamba2Block(p, dev)
    dec = blk.new_decode_state(R, dev)
    u_static = torch.zeros((R, 64), device=dev)
    g, out = blk.capture_step(u_static, dec)
    eager = {"state": dec["state"].clone(), "ring": dec["ring"].clone()}
    for rep in range(3):
        u = torch.from_numpy(rng.standard_normal((R, 64)).astype(np.float32)).to(dev)
        want = blk.step(u, eager)          # eager work between the replays
        torch.cuda.synchronize()
        u_static.copy_(u)
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(out.cpu().numpy(), want.cpu().numpy())
        np.testing.assert_array_equal(dec["state"].cpu().numpy(), eager["state"].cpu().numpy())


def test_mamba2_block_matches_reference_build(dev):
    """The block against Mamba2SSD::forward from a reference build (tests/golden/mamba2_ref.npz,
    the faithful path with x / z / out_proj packed ternary and B / C / dt float, two sequences
    of 19 tokens).  Every stage above is pinned on the GPU's own upstream tensors; end to end
    an fp32-level difference in the normed input can move an out_proj int8 code by one step,
    so the bound is one code step of the output scale (1/127) at most and 1e-3 on average."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "mamba2_ref.npz"),
                allow_pickle=False)
    p = {k: g[k].astype(np.float32) for k in g.files if not k.startswith(("u", "out", "shape"))}
    H, P, N, G = (int(v) for v in g["shape"])
    p.update(H=H, P=P, N=N, G=G)
    u = g["u"].astype(np.float32)
    b, s, d = u.shape
    blk = Mamba2Block(p, dev)
    cu = torch.tensor([0, s, 2 * s], dtype=torch.int32, device=dev)
    got = _np(blk.forward(torch.from_numpy(u.reshape(b * s, d)).to(dev), cu)["out"]).reshape(u.shape)
    want = g["out_packed"]
    scale = np.abs(want).max()
    err = np.abs(got - want)
    assert err.max() <= scale / 127, (err.max(), scale)
    assert err.mean() <= 1e-3 * scale, (err.mean(), scale)


@pytest.mark.parametrize("chunk", [0, 8])
def test_mamba2_block_matches_reference_build_d_state_64(dev, chunk):
    """The block at the reference's default d_state 64 (tests/golden/mamba2_n64_ref.npz:
    d_model 128, 4 heads of 64, 2 groups, two sequences of 41 tokens) against
    Mamba2SSD::forward from a reference build, through the sequential scan (chunk 0) and the
    time-chunked one (chunks of 8 tokens: carried states and conv windows across chunk
    boundaries), with the bound of the d_state 16 case above."""
    import os
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "mamba2_n64_ref.npz"),
                allow_pickle=False)
    p = {k: g[k].astype(np.float32) for k in g.files if not k.startswith(("u", "out", "shape"))}
    H, P, N, G = (int(v) for v in g["shape"])
    p.update(H=H, P=P, N=N, G=G)
    u = g["u"].astype(np.float32)
    b, s, d = u.shape
    blk = Mamba2Block(p, dev)
    cu = torch.tensor([0, s, 2 * s], dtype=torch.int32, device=dev)
    res = blk.forward(torch.from_numpy(u.reshape(b * s, d)).to(dev), cu, chunk_tokens=chunk)
    got = _np(res["out"]).reshape(u.shape)
    want = g["out_packed"]
    scale = np.abs(want).max()
    err = np.abs(got - want)
    assert err.max() <= scale / 127, (err.max(), scale)
    assert err.mean() <= 1e-3 * scale, (err.mean(), scale)


def _step_inputs(rng, dev, R, H, P, N, G, W, dtype):
    """Random projections (B / C / dt as column slices of one [R, 2*G*N + H] output, as the
    block produces them), a non-zero ring and state."""
    inner, gs = H * P, G * N
    cd = inner + 2 * gs
    t = lambda a, dt=torch.float32: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev, dt)
    sens = t(np.concatenate([rng.standard_normal((R, 2 * gs)),
                             rng.standard_normal((R, H)) - 1.0], 1), dtype)
    return {
        "x": t(rng.standard_normal((R, inner)), dtype), "z": t(rng.standard_normal((R, inner)), dtype),
        "B": sens[:, :gs], "C": sens[:, gs:2 * gs], "dt": sens[:, 2 * gs:],
        "conv_w": t(rng.standard_normal((cd, W)) * 0.5), "conv_b": t(rng.standard_normal(cd) * 0.1),
        "ring": t(rng.standard_normal((R, max(W - 1, 1), cd))),
        "a_log": t(rng.standard_normal(H)), "D": t(rng.standard_normal(H)),
        "norm_w": t(rng.uniform(0.5, 1.5, inner)),
        "state": t(rng.standard_normal((R, inner, N))),
    }


def _run_fused(ops, a, H, P, N, G):
    ring, state = a["ring"].clone(), a["state"].clone()
    W = a["conv_w"].shape[1]
    q, s, y = ops.mamba2_step(a["x"], a["z"], a["B"], a["C"], a["dt"], a["conv_w"], a["conv_b"],
                              ring if W > 1 else None, a["a_log"], a["D"], a["norm_w"], state,
                              H, P, N, G)
    return ring, state, y, q, s


@pytest.mark.parametrize("R,H,P,N,G,W,dtype", [
    (3, 8, 64, 16, 1, 4, torch.float32),      # inner 512: the norm's register path
    (2, 16, 64, 32, 2, 4, torch.bfloat16),
    (5, 8, 128, 64, 4, 3, torch.float32),
    (4, 4, 128, 4, 1, 2, torch.float32),
    (1, 32, 64, 16, 1, 4, torch.float32),     # the bench's block, one row
    (2, 3, 40, 8, 3, 4, torch.float32),       # inner 120: the norm sums in another order
    (6, 2, 24, 16, 1, 1, torch.bfloat16),     # no ring (width 1)
])
def test_mamba2_step_fused_equals_unfused_chain(dev, R, H, P, N, G, W, dtype):
    from reimagined_amd import ops
    rng = np.random.default_rng(R * 1000 + H * 10 + N)
    a = _step_inputs(rng, dev, R, H, P, N, G, W, dtype)
    inner, gs = H * P, G * N
    ring, state, y, q, s = _run_fused(ops, a, H, P, N, G)
    # the separate ops on separate copies of the ring's x / B / C slices
    rings = [a["ring"][:, :, lo:hi].contiguous() for lo, hi in
             ((0, inner), (inner, inner + gs), (inner + gs, inner + 2 * gs))]
    cw, cb = a["conv_w"], a["conv_b"]
    sl = ((0, inner), (inner, inner + gs), (inner + gs, inner + 2 * gs))
    xc, Bc, Cc = (ops.conv_step(v, cw[lo:hi].contiguous(), cb[lo:hi].contiguous(),
                                rg if W > 1 else None)
                  for v, rg, (lo, hi) in zip((a["x"], a["B"], a["C"]), rings, sl))
    st2 = a["state"].clone()
    y2 = ops.selective_scan_step(xc, a["dt"].contiguous(), a["a_log"], Bc, Cc, a["D"], None, st2,
                                 H, P, N, G)
    normed = ops.rmsnorm_gated(y2, a["z"], a["norm_w"], eps=1e-5)
    q2, s2 = ops.quantize_activations_bitnet(normed, bits=8)
    if W > 1:
        np.testing.assert_array_equal(ring.cpu().numpy(), torch.cat(rings, 2).cpu().numpy())
    np.testing.assert_array_equal(state.cpu().numpy(), st2.cpu().numpy())
    np.testing.assert_array_equal(y.float().cpu().numpy(), y2.float().cpu().numpy())
    q, q2 = q.cpu().numpy().astype(np.int32), q2.cpu().numpy().astype(np.int32)
    if inner % 512 == 0 and inner <= 4096:
        np.testing.assert_array_equal(q, q2)
        np.testing.assert_array_equal(s.cpu().numpy(), s2.cpu().numpy())
    else:
        # the row sum of squares in another order: the normed values agree to its rounding
        assert np.abs(q - q2).max() <= 1
        assert (q != q2).mean() <= 0.02
        np.testing.assert_allclose(s.cpu().numpy(), s2.cpu().numpy(), rtol=1e-5)


@pytest.mark.parametrize("R,H,P,N,G,W", [(3, 8, 64, 16, 1, 4), (2, 3, 40, 8, 3, 3),
                                         (2, 4, 32, 64, 2, 4)])
def test_mamba2_step_fused_matches_oracle(dev, orc, R, H, P, N, G, W):
    """Against the oracle's decode chain (conv_step, scan_step, rmsnorm_gated, quantize_act,
    src/mamba2.cpp:4072-4119 and src/bitlinear.cpp:240-291): ring exact; state and y within
    the fp32 bound; codes within one step where the normed value sits near a rounding
    boundary, act_scale within 1e-4."""
    from reimagined_amd import ops
    rng = np.random.default_rng(77 + N)
    a = _step_inputs(rng, dev, R, H, P, N, G, W, torch.float32)
    inner, gs = H * P, G * N
    ring, state, y, q, s = _run_fused(ops, a, H, P, N, G)
    h = {k: v.float().cpu().numpy() for k, v in a.items()}
    xBC = np.concatenate([h["x"], h["B"], h["C"]], 1)
    conv, ring_o = orc.conv_step(xBC, h["conv_w"], h["conv_b"], h["ring"])
    np.testing.assert_array_equal(ring.cpu().numpy(), ring_o)
    y_o, st_o = orc.scan_step(conv[:, :inner], h["dt"], h["a_log"], conv[:, inner:inner + gs],
                              conv[:, inner + gs:], h["D"], None, h["state"], H, P, N, G,
                              gate_silu=False)
    np.testing.assert_allclose(state.cpu().numpy(), st_o, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(y.cpu().numpy(), y_o, rtol=1e-4, atol=1e-5 * np.abs(y_o).max())
    normed = orc.rmsnorm_gated(y.cpu().numpy(), h["z"], h["norm_w"], eps=1e-5)
    q_o, s_o = orc.quantize_act(normed, 8)
    diff = np.abs(q.cpu().numpy().astype(np.int32) - q_o.astype(np.int32))
    assert diff.max() <= 1 and (diff > 0).mean() <= 0.02
    np.testing.assert_allclose(s.cpu().numpy(), s_o, rtol=1e-4)


def test_mamba2_step_rejects_unsupported_shapes(dev):
    """Shapes the fused launch does not take are refused (ValueError, as every rejected
    shape), as the reference's strict GPU step refuses a shape with no device path
    (src/mamba2.cpp:4031-4036)."""
    from reimagined_amd import ops
    rng = np.random.default_rng(1)
    a = _step_inputs(rng, dev, 1, 2, 16, 12, 1, 4, torch.float32)      # N = 12
    with pytest.raises(ValueError, match="N in"):
        _run_fused(ops, a, 2, 16, 12, 1)
    a = _step_inputs(rng, dev, 1, 2, 16, 16, 1, 5, torch.float32)      # width 5
    with pytest.raises(ValueError, match="conv_width"):
        _run_fused(ops, a, 2, 16, 16, 1)


@pytest.mark.parametrize("R,H,P,N,G,W,dtype,d", [
    (1, 32, 64, 16, 1, 4, torch.float32, 1024),   # the bench block: GEMV with the norm prologue
    (1, 8, 64, 16, 1, 4, torch.bfloat16, 256),
    (1, 3, 48, 8, 3, 4, torch.float32, 64),       # inner 144 (not % 64): norm launch + GEMM
    (3, 8, 64, 32, 2, 3, torch.float32, 128),     # three rows: norm launch + GEMM
])
def test_mamba2_step_out_equals_step_then_gemm(dev, R, H, P, N, G, W, dtype, d):
    """nsosx_mamba2_step_out equals nsosx_mamba2_step followed by the out_proj ternary GEMM
    on its codes, bit for bit: out, codes, act_scale, state, ring and y."""
    from reimagined_amd import ops
    rng = np.random.default_rng(R * 100 + H + d)
    a = _step_inputs(rng, dev, R, H, P, N, G, W, dtype)
    inner = H * P
    w = rng.standard_normal((d, inner)).astype(np.float32)
    packed, ws = ops.pack_ternary(w)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    mag = torch.from_numpy(rng.uniform(0.5, 1.5, d).astype(np.float32)).to(dev)
    res = []
    for fused in (False, True):
        ring, state = a["ring"].clone(), a["state"].clone()
        q = torch.empty((R, inner), dtype=torch.int8, device=dev)
        s = torch.empty(R, dtype=torch.float32, device=dev)
        out = torch.empty((R, d), dtype=dtype, device=dev)
        kw = dict(q=q, act_scale=s)
        if fused:
            kw.update(out_proj=(pk, ws, mag, None), out=out)
        _, _, y = ops.mamba2_step(a["x"], a["z"], a["B"], a["C"], a["dt"], a["conv_w"],
                                  a["conv_b"], ring if W > 1 else None, a["a_log"], a["D"],
                                  a["norm_w"], state, H, P, N, G, **kw)
        if not fused:
            out = ops.ternary_gemm(q, s, pk, ws, d, magnitude=mag, out_dtype=dtype)
        torch.cuda.synchronize()
        res.append([t.float().cpu().numpy() for t in (out, q, s, state, ring, y)])
    for want, got in zip(*res):
        np.testing.assert_array_equal(got, want)
