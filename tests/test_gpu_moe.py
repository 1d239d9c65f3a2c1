"""Top-k MoE routing, grouped ternary GEMMs and the combine on the GPU against the
CPU oracle.  Selections, counts, offsets and the permutation are bit-exact;
routing weights within 1e-6 relative (GPU and host expf may differ by an ulp);
expert outputs bit-exact given the same activation codes."""
import numpy as np
import pytest
import torch

from reimagined_amd import ops
from reimagined_amd.layers import MoEFFN

pytestmark = pytest.mark.gpu


def _route_oracle(orc, logits, k):
    probs = orc.softmax_rows(logits)
    w, sel = orc.topk_mask(probs, k)
    counts, offsets, perm = orc.moe_dispatch(probs, k)
    return w, sel, counts, offsets, perm


@pytest.mark.parametrize("rows,E,k", [(8192, 8, 2), (1, 8, 2), (300, 8, 1), (1000, 64, 8),
                                      (513, 3, 3), (700, 16, 12), (300, 64, 64), (4000, 32, 9)])
def test_route_matches_oracle(dev, orc, rows, E, k):
    rng = np.random.default_rng(rows + E)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    r = ops.moe_route(torch.from_numpy(logits).to(dev), k)
    w, sel, counts, offsets, perm = _route_oracle(orc, logits, k)
    np.testing.assert_array_equal(r["selected"].cpu().numpy(), sel)
    np.testing.assert_array_equal(r["counts"].cpu().numpy(), counts)
    np.testing.assert_array_equal(r["offsets"].cpu().numpy(), offsets)
    np.testing.assert_array_equal(r["perm"].cpu().numpy(), perm)
    np.testing.assert_allclose(r["weights"].cpu().numpy(), w, rtol=1e-6, atol=1e-7)
    slot_of = r["slot_of"].cpu().numpy()
    pm = r["perm"].cpu().numpy()
    for i in range(k):  # slot_of is the inverse map of perm, in rank order
        np.testing.assert_array_equal(pm[slot_of[:, i]], np.arange(rows))
        seg = np.searchsorted(offsets, slot_of[:, i], side="right") - 1
        np.testing.assert_array_equal(seg, sel[:, i])


@pytest.mark.parametrize("rows,E,k", [(1, 8, 2), (37, 16, 4)])
def test_route_select_only_matches_full(dev, rows, E, k):
    rng = np.random.default_rng(rows * 3 + E)
    logits = torch.from_numpy(rng.standard_normal((rows, E)).astype(np.float32)).to(dev)
    full = ops.moe_route(logits, k)
    sel = ops.moe_route(logits, k, select_only=True)
    assert set(sel) == {"weights", "selected"}
    torch.testing.assert_close(sel["selected"], full["selected"], rtol=0, atol=0)
    torch.testing.assert_close(sel["weights"], full["weights"], rtol=0, atol=0)


def test_route_partial_null_outputs_rejected(dev):
    logits = torch.zeros((4, 8), dtype=torch.float32, device=dev)
    w = torch.empty((4, 8), dtype=torch.float32, device=dev)
    s = torch.empty((4, 2), dtype=torch.int32, device=dev)
    counts = torch.empty(8, dtype=torch.int32, device=dev)
    rc = ops.lib().nsosx_moe_route(logits.data_ptr(), None, 4, 8, 2, w.data_ptr(),
                                   s.data_ptr(), counts.data_ptr(), None, None, None, None, None,
                                   None)
    assert rc != 0
    assert b"null pointer" in ops.lib().nsosx_last_error()


@pytest.mark.parametrize("rows,E,k", [(8192, 8, 2), (1000, 64, 8), (300, 8, 1), (900, 32, 9),
                                      (300, 16, 16)])
def test_route_padding_rows_match_oracle(dev, orc, rows, E, k):
    """MoERouter::forward(x, valid_rows): padding rows get zero weights, selections -1,
    slot_of -1 and no slots; the rest route as without the mask.  loads = expert_loads."""
    rng = np.random.default_rng(3 * rows + E)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    valid = (rng.random(rows) < 0.75).astype(np.uint8)
    valid[-1] = 0
    r = ops.moe_route(torch.from_numpy(logits).to(dev), k, valid_rows=valid, want_loads=True)
    w, sel = orc.topk_mask(orc.softmax_rows(logits), k, valid)
    counts, offsets, perm = orc.moe_dispatch_sel(sel, E)
    np.testing.assert_array_equal(r["selected"].cpu().numpy(), sel)
    np.testing.assert_array_equal(r["counts"].cpu().numpy(), counts)
    np.testing.assert_array_equal(r["offsets"].cpu().numpy(), offsets)
    n = int(offsets[-1])
    assert n == int(valid.sum()) * k
    np.testing.assert_array_equal(r["perm"].cpu().numpy()[:n], perm[:n])
    gw = r["weights"].cpu().numpy()
    np.testing.assert_allclose(gw, w, rtol=1e-6, atol=1e-7)
    assert np.all(gw[valid == 0] == 0.0)
    slot_of = r["slot_of"].cpu().numpy()
    assert np.all(slot_of[valid == 0] == -1)
    pm = r["perm"].cpu().numpy()
    idx = np.flatnonzero(valid)
    for i in range(k):
        np.testing.assert_array_equal(pm[slot_of[idx, i]], idx)
    # the device loads sum the device weights in the oracle's order: bit-exact on them
    np.testing.assert_array_equal(r["loads"].cpu().numpy(), orc.expert_loads(gw, valid))
    np.testing.assert_allclose(r["loads"].cpu().numpy(), orc.expert_loads(w, valid), rtol=1e-5)


def test_route_loads_without_mask_select_only(dev, orc):
    rng = np.random.default_rng(77)
    logits = torch.from_numpy(rng.standard_normal((777, 8)).astype(np.float32)).to(dev)
    r = ops.moe_route(logits, 2, select_only=True, want_loads=True)
    np.testing.assert_array_equal(r["loads"].cpu().numpy(),
                                  orc.expert_loads(r["weights"].cpu().numpy()))


def test_route_mask_checked_on_host(dev):
    logits = torch.zeros((4, 8), dtype=torch.float32, device=dev)
    with pytest.raises(ValueError, match="only 0 or 1"):
        ops.moe_route(logits, 2, valid_rows=np.array([1, 2, 1, 1], np.uint8))
    with pytest.raises(ValueError, match="size mismatch"):
        ops.moe_route(logits, 2, valid_rows=np.array([1, 1, 1], np.uint8))


def test_route_ties_prefer_lower_index(dev, orc):
    logits = np.zeros((4, 8), np.float32)
    logits[1, [2, 5]] = 1.0
    logits[2, [7, 6, 0]] = [3.0, 3.0, 3.0]
    logits[3] = np.arange(8, dtype=np.float32)[::-1].copy()
    r = ops.moe_route(torch.from_numpy(logits).to(dev), 2)
    sel = r["selected"].cpu().numpy()
    assert sel.tolist() == [[0, 1], [2, 5], [0, 6], [0, 1]]
    w = r["weights"].cpu().numpy()
    assert np.all((w > 0).sum(axis=1) == 2)
    np.testing.assert_allclose(w.sum(axis=1), 1.0, atol=1e-6)


def _ternary(rng, n, k):
    return rng.standard_normal((n, k)).astype(np.float32)


@pytest.mark.parametrize("hidden_dtype,E,k", [(torch.float32, 8, 2), (torch.float32, 16, 10),
                                               (torch.float32, 12, 12)])
def test_moe_ffn_matches_oracle(dev, orc, hidden_dtype, E, k):
    """The whole MoE feed-forward (routing, grouped up / squared ReLU / down GEMMs, combine)
    against the oracle's per-expert BitLinear chain: top-2 of 8, top-10 of 16 (wider than the
    register fast paths) and k = E = 12 (every row through every expert, raw softmax weights)."""
    rng = np.random.default_rng(77 + k)
    rows, d, f = 600, 256, 512
    w_up = [_ternary(rng, f, d) for _ in range(E)]
    w_down = [_ternary(rng, d, f) for _ in range(E)]
    x = rng.standard_normal((rows, d)).astype(np.float32)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    moe = MoEFFN(w_up, w_down, dev, k=k, rms_input=True, hidden_dtype=hidden_dtype)
    out = moe.forward(torch.from_numpy(x).to(dev), torch.from_numpy(logits).to(dev),
                      out_dtype=torch.float32)
    w, sel, counts, offsets, perm = _route_oracle(orc, logits, k)
    np.testing.assert_array_equal(out["perm"].cpu().numpy(), perm)
    # per-expert BitLinear chain on the oracle, slot order
    h_want = np.zeros((rows * k, f), np.float32)
    o_want = np.zeros((rows * k, d), np.float32)
    for e in range(E):
        rs = perm[offsets[e]:offsets[e + 1]]
        if rs.size == 0:
            continue
        pu, wsu, _ = orc.pack_weights(w_up[e])
        pd, wsd, _ = orc.pack_weights(w_down[e])
        hu = orc.bitlinear_forward(x[rs], pu, wsu, f, rms_input=True)
        hu = orc.squared_relu(hu)
        h_want[offsets[e]:offsets[e + 1]] = hu
        o_want[offsets[e]:offsets[e + 1]] = orc.bitlinear_forward(hu, pd, wsd, d, rms_input=True)
    np.testing.assert_array_equal(out["h"].cpu().numpy(), h_want)
    np.testing.assert_array_equal(out["o"].cpu().numpy(), o_want)
    want = orc.moe_combine(o_want, perm, offsets, out["weights"].cpu().numpy())
    np.testing.assert_array_equal(out["out"].cpu().numpy(), want)
    # against the oracle's own routing weights: fp32 tolerance scaled to the output
    # (two products summed can cancel, so a per-element relative bound is not meaningful)
    want_w = orc.moe_combine(o_want, perm, offsets, w)
    got = out["out"].cpu().numpy()
    np.testing.assert_allclose(got, want_w, rtol=1e-4, atol=1e-5 * np.abs(want_w).max())


@pytest.mark.parametrize("in_dt,out_dt", [(torch.float32, torch.float32),
                                           (torch.bfloat16, torch.float32),
                                           (torch.float32, torch.bfloat16),
                                           (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("rows,E,k,dim", [(300, 8, 2, 1024), (77, 8, 3, 1022), (1, 4, 1, 8),
                                          (70000, 8, 2, 64), (200, 16, 12, 1024),
                                          (50, 64, 64, 520), (33, 32, 9, 1022)])
def test_moe_combine_matches_oracle(dev, orc, in_dt, out_dt, rows, E, k, dim):
    """The weighted combine alone, both input and output dtypes, the row-per-wave vector form
    (dim % 4 == 0) and the element-wise one (dim = 1022), over the device routing: bit-exact
    with the oracle's ascending-expert sum (a bf16 output is that sum rounded to nearest even).
    70000 rows exceed the element-wise form's 65535-row grid limit."""
    rng = np.random.default_rng(rows * 7 + dim + k)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    r = ops.moe_route(torch.from_numpy(logits).to(dev), k)
    o = torch.from_numpy(rng.standard_normal((rows * k, dim)).astype(np.float32)).to(in_dt)
    got = ops.moe_combine(o.to(dev), r["slot_of"], r["selected"], r["weights"], out_dtype=out_dt)
    want = orc.moe_combine(o.float().numpy(), r["perm"].cpu().numpy(), r["offsets"].cpu().numpy(),
                           r["weights"].cpu().numpy())
    want_t = torch.from_numpy(want).to(out_dt)
    assert torch.equal(got.cpu(), want_t)


@pytest.mark.parametrize("rows,E,k", [(1, 8, 2), (5, 8, 2), (32, 8, 2), (5, 16, 10)])
def test_moe_sparse_decode_matches_oracle(dev, orc, rows, E, k):
    """Decode rows through (row, routed expert) grouped GEMVs: bit-exact against the oracle's
    per-expert BitLinear chain combined with the same routing weights (also top-10 of 16)."""
    rng = np.random.default_rng(90 + rows + k)
    d, f = 256, 512
    w_up = [_ternary(rng, f, d) for _ in range(E)]
    w_down = [_ternary(rng, d, f) for _ in range(E)]
    x = rng.standard_normal((rows, d)).astype(np.float32)
    logits = rng.standard_normal((rows, E)).astype(np.float32)
    moe = MoEFFN(w_up, w_down, dev, k=k, rms_input=True)
    res = moe.decode(torch.from_numpy(x).to(dev), torch.from_numpy(logits).to(dev),
                     out_dtype=torch.float32)
    w_gpu = res["weights"].cpu().numpy()
    sel = res["selected"].cpu().numpy()
    packs_u = [orc.pack_weights(w) for w in w_up]
    packs_d = [orc.pack_weights(w) for w in w_down]
    want = np.zeros((rows, d), np.float32)
    for r in range(rows):
        acc = np.float32(0.0) * np.zeros(d, np.float32)
        for e in sorted(sel[r]):
            pu, wsu, _ = packs_u[e]
            pd, wsd, _ = packs_d[e]
            h = orc.squared_relu(orc.bitlinear_forward(x[r:r + 1], pu, wsu, f, rms_input=True))
            o = orc.bitlinear_forward(h, pd, wsd, d, rms_input=True)[0]
            acc = (acc + (o * w_gpu[r, e]).astype(np.float32)).astype(np.float32)
        want[r] = acc
    np.testing.assert_array_equal(res["out"].cpu().numpy(), want)
    w_orc, sel_orc = orc.topk_mask(orc.softmax_rows(logits), k)
    np.testing.assert_array_equal(sel, sel_orc)


@pytest.mark.parametrize("hidden_dtype", [torch.float32, torch.bfloat16])
def test_moe_ffn_padding_rows(dev, hidden_dtype):
    """forward_moe over a padded batch (valid_rows from the batch's valid lengths,
    src/jamba.cpp:3708-3710): the valid rows come out bit for bit as a forward over the
    valid rows alone, the padding rows as zeros, and no expert slot holds a padding row."""
    rng = np.random.default_rng(81)
    rows, E, k, d, f = 700, 8, 2, 256, 512
    w_up = [_ternary(rng, f, d) for _ in range(E)]
    w_down = [_ternary(rng, d, f) for _ in range(E)]
    x = torch.from_numpy(rng.standard_normal((rows, d)).astype(np.float32)).to(dev)
    logits = torch.from_numpy(rng.standard_normal((rows, E)).astype(np.float32)).to(dev)
    valid = (rng.random(rows) < 0.6).astype(np.uint8)
    idx = torch.from_numpy(np.flatnonzero(valid)).to(dev)
    moe = MoEFFN(w_up, w_down, dev, k=k, rms_input=True, hidden_dtype=hidden_dtype)
    got = moe.forward(x, logits, out_dtype=torch.float32, valid_rows=valid)
    out = got["out"].clone()
    n = int(got["offsets"][-1])
    assert n == int(valid.sum()) * k
    assert set(got["perm"][:n].cpu().numpy().tolist()) <= set(idx.cpu().numpy().tolist())
    ref = moe.forward(x[idx].contiguous(), logits[idx].contiguous(), out_dtype=torch.float32)
    assert torch.equal(out[idx], ref["out"])
    assert torch.count_nonzero(out[torch.from_numpy(valid == 0).to(dev)]) == 0
    # a device mask reads the same
    got2 = moe.forward(x, logits, out_dtype=torch.float32,
                       valid_rows=torch.from_numpy(valid).to(dev))
    assert torch.equal(got2["out"], out)


def test_moe_sparse_decode_padding_rows(dev):
    """Sparse decode with padding rows: they take no expert GEMV and come out as zeros; the
    valid rows equal a decode of the valid rows alone."""
    rng = np.random.default_rng(82)
    rows, E, k, d, f = 9, 8, 2, 256, 512
    w_up = [_ternary(rng, f, d) for _ in range(E)]
    w_down = [_ternary(rng, d, f) for _ in range(E)]
    x = torch.from_numpy(rng.standard_normal((rows, d)).astype(np.float32)).to(dev)
    logits = torch.from_numpy(rng.standard_normal((rows, E)).astype(np.float32)).to(dev)
    valid = np.array([1, 0, 1, 1, 0, 0, 1, 1, 0], np.uint8)
    idx = torch.from_numpy(np.flatnonzero(valid)).to(dev)
    moe = MoEFFN(w_up, w_down, dev, k=k, rms_input=True)
    out = moe.decode(x, logits, out_dtype=torch.float32, valid_rows=valid)["out"].clone()
    ref = moe.decode(x[idx].contiguous(), logits[idx].contiguous(), out_dtype=torch.float32)
    assert torch.equal(out[idx], ref["out"])
    assert torch.count_nonzero(out[torch.from_numpy(valid == 0).to(dev)]) == 0


def test_moe_ffn_full_size_sampled(dev, orc):
    """Config 5's MoE prefill at full size (8192 bf16 tokens, 8 experts of 1024 -> 4096 -> 1024,
    top-2, bf16 hidden), the shapes the bench times: the permutation bit-exact, and for
    sampled slots the up projection (bf16 of the oracle's squared-ReLU output) and the down
    projection (on the GPU's hidden row) bit-exact, and sampled combined rows bit-exact with
    the oracle's ascending-expert sum over the GPU's expert outputs."""
    from reimagined_amd import workloads
    moe_p, _ = workloads.config5(rows=8192, decode_rows=1, d_inner=64)
    E, k = 8, 2
    moe = MoEFFN(moe_p["w_up"], moe_p["w_down"], dev, k=k, rms_input=True,
                 hidden_dtype=torch.bfloat16)
    xb = torch.from_numpy(moe_p["x"]).to(torch.bfloat16)
    logits = moe_p["logits"]
    res = moe.forward(xb.to(dev), torch.from_numpy(logits).to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    _, _, _, offsets, perm = _route_oracle(orc, logits, k)
    np.testing.assert_array_equal(res["perm"].cpu().numpy(), perm)
    np.testing.assert_array_equal(res["offsets"].cpu().numpy(), offsets)
    h = res["h"]
    o = res["o"]
    xf = xb.float().numpy()
    rng = np.random.default_rng(505)
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        slots = np.unique(np.concatenate([rng.choice(np.arange(lo, hi), 12, replace=False),
                                          [lo, hi - 1]]))
        pu, wsu, _ = orc.pack_weights(moe_p["w_up"][e])
        pd, wsd, _ = orc.pack_weights(moe_p["w_down"][e])
        hu = orc.squared_relu(orc.bitlinear_forward(xf[perm[slots]], pu, wsu, 4096, rms_input=True))
        ts = torch.from_numpy(slots).to(dev)
        h_gpu = h[ts].float().cpu().numpy()
        np.testing.assert_array_equal(h_gpu, torch.from_numpy(hu).to(torch.bfloat16).float().numpy())
        od = orc.bitlinear_forward(h_gpu, pd, wsd, 1024, rms_input=True)
        np.testing.assert_array_equal(o[ts].cpu().numpy(), od)
    rows = np.unique(rng.choice(8192, 64, replace=False))
    want = orc.moe_combine(o.cpu().numpy(), perm, offsets, res["weights"].cpu().numpy())
    np.testing.assert_array_equal(res["out"].cpu().numpy()[rows], want[rows])


@pytest.mark.parametrize("gather,sqrelu,out_dtype", [(True, True, torch.bfloat16),
                                                     (False, False, torch.float32),
                                                     (True, False, torch.float32),
                                                     (False, True, torch.bfloat16)])
def test_grouped_gemm_segments(dev, orc, gather, sqrelu, out_dtype):
    """The grouped ternary GEMM over constructed expert segments: empty experts, a single row,
    segments across one and several 128-row tiles, N with an edge tile (520) and K = 384
    (three ring stages), with magnitude and bias; each segment bit-exact against the oracle's
    dequantized product (squared ReLU, bf16 RNE where asked)."""
    rng = np.random.default_rng(11 + 2 * gather + sqrelu)
    counts = [0, 1, 129, 0, 300, 64, 257]
    E, K, N = len(counts), 384, 520
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    slots = int(offsets[-1])
    rows = slots + 17
    q = rng.integers(-127, 128, size=(rows, K), dtype=np.int8)
    s = rng.uniform(0.001, 0.02, rows).astype(np.float32)
    perm = rng.permutation(rows)[:slots].astype(np.int32) if gather else np.arange(slots, dtype=np.int32)
    ws_, packs, codes, mags, biases = [], [], [], [], []
    entries = []
    for e in range(E):
        pk, wsc, cd = orc.pack_weights(rng.standard_normal((N, K)).astype(np.float32))
        mg = rng.uniform(0.5, 1.5, N).astype(np.float32)
        bs = rng.standard_normal(N).astype(np.float32)
        pk_t = torch.from_numpy(pk.view(np.int32)).to(dev)
        entries.append((pk_t, wsc, K, N, torch.from_numpy(mg).to(dev), torch.from_numpy(bs).to(dev)))
        ws_.append(wsc); codes.append(cd); mags.append(mg); biases.append(bs)
    views = ops.LinearViewArray(entries, dev)
    qd, sd = torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev)
    offd, permd = torch.from_numpy(offsets).to(dev), torch.from_numpy(perm).to(dev)
    # compact (the real row tiles from the offsets) and the full per-expert grid
    total = slots if (gather + sqrelu) % 2 == 0 else 0
    if gather:
        y = ops.grouped_ternary_gemm(views, offd, permd, qd, sd, N, max(counts), sqrelu, True,
                                     out_dtype, total_rows=total)
    else:
        y = ops.grouped_ternary_gemm(views, offd, None, qd[:slots], sd[:slots], N, max(counts),
                                     sqrelu, False, out_dtype, total_rows=total)
    got = y.float().cpu().numpy()
    for e in range(E):
        lo, hi = int(offsets[e]), int(offsets[e + 1])
        if hi == lo:
            continue
        src = perm[lo:hi]
        want = orc.dequant(orc.gemm_i8(q[src], codes[e]), s[src], ws_[e], mags[e], biases[e])
        if sqrelu:
            want = orc.squared_relu(want)
        if out_dtype == torch.bfloat16:
            want = torch.from_numpy(want).to(torch.bfloat16).float().numpy()
        np.testing.assert_array_equal(got[lo:hi], want, err_msg=f"expert {e}")
