"""Pins the selective-scan and MoE parts of the CPU oracle (CPU only).

The scan is checked against the explicit closed form of the linear recurrence
(h_t = sum_s prod_{u>s} a_u * b_s, evaluated in float64), against invariants
that reduce it to a cumulative sum or to the D skip, against per-sequence
decomposition of a packed ragged batch, and step == last row of the prefill
(OXN/nsos/src/mamba2.cpp:2814-2818 relies on that equivalence).  The router is
checked against the structural invariants of
OXN/nsos/tests/gpu/test_gpu_parity_moe_router.cpp:100-152 and constructed ties.
"""
import math

import numpy as np
import pytest


def _scan_inputs(rng, T, H, P, N, G, per_state=True):
    D = H * P
    x = rng.standard_normal((T, D)).astype(np.float32)
    dt = rng.normal(-2.0, 0.5, (T, H)).astype(np.float32)
    a_log = rng.standard_normal((H, N) if per_state else (H,)).astype(np.float32)
    B = (rng.standard_normal((T, G * N)) * 0.25).astype(np.float32)
    C = (rng.standard_normal((T, G * N)) * 0.25).astype(np.float32)
    Dk = rng.standard_normal(H).astype(np.float32)
    z = rng.standard_normal((T, D)).astype(np.float32)
    return x, dt, a_log, B, C, Dk, z


def _closed_form(orc, x, dt, a_log, B, C, Dk, z, H, P, N, G, gate=True):
    T, D = x.shape
    y = np.zeros((T, D))
    state = np.zeros((D, N))
    for h in range(H):
        g = (h * G) // H
        for p in range(P):
            ch = h * P + p
            a = np.zeros((T, N))
            b = np.zeros((T, N))
            for t in range(T):
                for n in range(N):
                    al = a_log[h, n] if a_log.ndim == 2 else a_log[h]
                    delta, decay = orc.decay_terms(float(dt[t, h]), float(al))
                    a[t, n] = decay
                    b[t, n] = delta * float(B[t, g * N + n]) * float(x[t, ch])
            for t in range(T):
                hs = np.zeros(N)
                for s in range(t + 1):
                    hs += np.prod(a[s + 1:t + 1], axis=0) * b[s]
                out = float(Dk[h]) * float(x[t, ch]) + float(np.dot(hs, C[t, g * N:(g + 1) * N]))
                if gate:
                    zz = float(z[t, ch])
                    out *= zz / (1.0 + math.exp(-zz))
                y[t, ch] = out
                if t == T - 1:
                    state[ch] = hs
    return y, state


@pytest.mark.parametrize("H,P,N,G,per_state", [(6, 1, 4, 1, True), (4, 2, 3, 2, False),
                                               (4, 2, 5, 4, True)])
def test_scan_matches_closed_form(orc, H, P, N, G, per_state):
    rng = np.random.default_rng(11)
    T = 9
    x, dt, a_log, B, C, Dk, z = _scan_inputs(rng, T, H, P, N, G, per_state)
    y, fin = orc.selective_scan(x, dt, a_log, B, C, Dk, z, [0, T], H, P, N, G)
    y_ref, st_ref = _closed_form(orc, x, dt, a_log, B, C, Dk, z, H, P, N, G)
    np.testing.assert_allclose(y, y_ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(fin[0], st_ref, rtol=1e-5, atol=1e-6)


def test_decay_terms_formula_and_edges(orc):
    for dt in (-3.0, -0.2, 0.0, 1.7, 19.0):
        for a in (-1.0, 0.0, 0.8):
            delta, decay = orc.decay_terms(dt, a)
            sp = math.log1p(math.exp(dt))
            assert delta == pytest.approx(sp, rel=1e-6)
            assert decay == pytest.approx(math.exp(-sp * math.exp(a)), rel=1e-6, abs=1e-30)
    assert orc.decay_terms(25.0, 0.0)[0] == 25.0            # softplus identity branch
    d, _ = orc.decay_terms(-30.0, 0.0)
    assert d == pytest.approx(math.exp(-30.0), rel=1e-6)    # exp branch
    assert orc.decay_terms(30.0, 30.0)[1] == 0.0              # log_q > 50 -> 0
    assert math.isnan(orc.decay_terms(float("nan"), 0.0)[1])
    assert math.isnan(orc.decay_terms(0.0, float("inf"))[1])


def test_scan_pure_accumulator_when_decay_is_one(orc):
    rng = np.random.default_rng(12)
    T, H, N = 40, 3, 4
    x, dt, _, B, C, Dk, z = _scan_inputs(rng, T, H, 1, N, 1)
    a_log = np.full((H, N), -80.0, np.float32)     # q ~ 0 -> decay == 1
    y, fin = orc.selective_scan(x, dt, a_log, B, C, Dk, None, [0, T], H, 1, N, 1, gate_silu=False)
    delta = np.array([[orc.decay_terms(float(v), -80.0)[0] for v in row] for row in dt])
    bx = delta[:, :, None] * B[:, None, :].astype(np.float64) * x[:, :, None]
    hist = np.cumsum(bx, axis=0)
    y_ref = Dk[None, :] * x + np.einsum("thn,tn->th", hist, C.astype(np.float64))
    np.testing.assert_allclose(y, y_ref, rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(fin[0], hist[-1], rtol=2e-5, atol=2e-6)


def test_scan_zero_delta_is_skip_only(orc):
    rng = np.random.default_rng(13)
    T, H, N = 12, 5, 3
    x, _, a_log, B, C, Dk, _ = _scan_inputs(rng, T, H, 1, N, 1)
    dt = np.full((T, H), -120.0, np.float32)      # softplus -> exp(-120) == 0 in float
    y, fin = orc.selective_scan(x, dt, a_log, B, C, Dk, None, [0, T], H, 1, N, 1, gate_silu=False)
    np.testing.assert_array_equal(y, (Dk[None, :] * x).astype(np.float32))
    assert np.all(fin == 0)


def test_scan_varlen_equals_per_sequence(orc):
    rng = np.random.default_rng(14)
    H, P, N, G = 4, 2, 4, 2
    lens = [5, 1, 9, 3]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    x, dt, a_log, B, C, Dk, z = _scan_inputs(rng, T, H, P, N, G)
    h0 = (rng.standard_normal((len(lens), H * P, N)) * 0.1).astype(np.float32)
    y, fin = orc.selective_scan(x, dt, a_log, B, C, Dk, z, cu, H, P, N, G, initial_state=h0)
    for s in range(len(lens)):
        a, b = cu[s], cu[s + 1]
        ys, fs = orc.selective_scan(x[a:b], dt[a:b], a_log, B[a:b], C[a:b], Dk, z[a:b],
                                    [0, b - a], H, P, N, G, initial_state=h0[s:s + 1])
        np.testing.assert_array_equal(y[a:b], ys)
        np.testing.assert_array_equal(fin[s], fs[0])


def test_scan_chaining_and_step_equal_full_scan(orc):
    rng = np.random.default_rng(15)
    H, P, N, G, T = 3, 2, 4, 1, 11
    x, dt, a_log, B, C, Dk, z = _scan_inputs(rng, T, H, P, N, G)
    y, fin = orc.selective_scan(x, dt, a_log, B, C, Dk, z, [0, T], H, P, N, G)
    y1, f1 = orc.selective_scan(x[:7], dt[:7], a_log, B[:7], C[:7], Dk, z[:7], [0, 7], H, P, N, G)
    y2, f2 = orc.selective_scan(x[7:], dt[7:], a_log, B[7:], C[7:], Dk, z[7:], [0, T - 7], H, P, N,
                                G, initial_state=f1)
    np.testing.assert_array_equal(np.concatenate([y1, y2]), y)
    np.testing.assert_array_equal(f2, fin)
    _, f_prefix = orc.selective_scan(x[:T - 1], dt[:T - 1], a_log, B[:T - 1], C[:T - 1], Dk,
                                     z[:T - 1], [0, T - 1], H, P, N, G)
    ys, st = orc.scan_step(x[T - 1:], dt[T - 1:], a_log, B[T - 1:], C[T - 1:], Dk, z[T - 1:],
                           f_prefix, H, P, N, G)
    np.testing.assert_array_equal(ys[0], y[T - 1])
    np.testing.assert_array_equal(st, fin)


def test_conv1d_matches_numpy_per_sequence(orc):
    rng = np.random.default_rng(16)
    Cn, W = 6, 4
    lens = [2, 7, 1, 5]
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    x = rng.standard_normal((int(cu[-1]), Cn)).astype(np.float32)
    w = rng.standard_normal((Cn, W)).astype(np.float32)
    b = rng.standard_normal(Cn).astype(np.float32)
    out = orc.conv1d_causal(x, w, cu, bias=b, silu_act=False)
    for s in range(len(lens)):
        seg = x[cu[s]:cu[s + 1]].astype(np.float64)
        for c in range(Cn):
            full = np.convolve(seg[:, c], w[c, ::-1].astype(np.float64))[:len(seg)] + b[c]
            np.testing.assert_allclose(out[cu[s]:cu[s + 1], c], full, rtol=1e-5, atol=1e-6)
    act = orc.conv1d_causal(x, w, cu, bias=b, silu_act=True)
    np.testing.assert_allclose(act, out / (1 + np.exp(-out.astype(np.float64))), rtol=1e-5, atol=1e-6)


def test_silu_softplus_squared_relu(orc):
    for v in (-30.0, -2.0, -0.1, 0.0, 0.3, 4.0, 30.0):
        assert orc.silu(v) == pytest.approx(v / (1 + math.exp(-v)), rel=1e-6, abs=1e-30)
        assert orc.softplus(v) == pytest.approx(math.log1p(math.exp(v)), rel=1e-6)
    x = np.array([-2, -0.0, 0.5, 3], np.float32)
    np.testing.assert_array_equal(orc.squared_relu(x), np.array([0, 0, 0.25, 9], np.float32))


def test_softmax_rows(orc):
    rng = np.random.default_rng(21)
    lg = rng.standard_normal((64, 8)).astype(np.float32)
    p = orc.softmax_rows(lg)
    e = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
    np.testing.assert_allclose(p, e / e.sum(axis=1, keepdims=True), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("experts,k", [(8, 2), (8, 1), (65, 2), (5, 4)])
def test_topk_mask_invariants(orc, experts, k):
    rng = np.random.default_rng(22)
    p = orc.softmax_rows(rng.standard_normal((200, experts)).astype(np.float32))
    w, sel = orc.topk_mask(p, k)
    assert np.all((w != 0).sum(axis=1) == k)
    assert np.all(np.abs(w.sum(axis=1) - 1) <= 1e-4)
    order = np.lexsort((np.arange(experts)[None, :].repeat(200, 0), -p), axis=1)[:, :k]
    np.testing.assert_array_equal(sel, order)


def test_topk_ties_prefer_lower_index(orc):
    p = np.array([[0.2, 0.3, 0.3, 0.2], [0.25, 0.25, 0.25, 0.25]], np.float32)
    w, sel = orc.topk_mask(p, 2)
    assert sel.tolist() == [[1, 2], [0, 1]]
    assert w[1].tolist() == [0.5, 0.5, 0.0, 0.0]


def test_dispatch_closed_form(orc):
    rng = np.random.default_rng(23)
    rows, E, k = 300, 8, 2
    p = orc.softmax_rows(rng.standard_normal((rows, E)).astype(np.float32))
    w, sel = orc.topk_mask(p, k)
    counts, offsets, perm = orc.moe_dispatch(w, k)
    for e in range(E):
        want = [r for r in range(rows) if e in sel[r]]
        assert counts[e] == len(want)
        assert perm[offsets[e]:offsets[e + 1]].tolist() == want
    assert offsets[0] == 0 and offsets[-1] == rows * k
    assert sorted(perm.tolist()) == sorted(list(range(rows)) * k)


def test_combine_expert_ascending(orc):
    rng = np.random.default_rng(24)
    rows, E, k, dim = 50, 4, 2, 6
    p = orc.softmax_rows(rng.standard_normal((rows, E)).astype(np.float32))
    w, _ = orc.topk_mask(p, k)
    counts, offsets, perm = orc.moe_dispatch(w, k)
    eo = rng.standard_normal((rows * k, dim)).astype(np.float32)
    out = orc.moe_combine(eo, perm, offsets, w)
    want = np.zeros((rows, dim), np.float32)
    for e in range(E):
        for s in range(offsets[e], offsets[e + 1]):
            want[perm[s]] = (want[perm[s]] + eo[s] * w[perm[s], e]).astype(np.float32)
    np.testing.assert_array_equal(out, want)


# ---- padding rows (MoERouter::forward(x, valid_rows), src/jamba.cpp:8140-8319) --------

@pytest.mark.parametrize("rows,E,k", [(300, 8, 2), (64, 16, 4), (7, 8, 8)])
def test_padding_rows_are_absent_from_dispatch(orc, rows, E, k):
    """Masked routing equals routing the valid rows alone, with the row ids mapped back:
    padding rows take no slot (the device dispatch counts only nonzero weights,
    src/cuda/moe_kernels.cu:226-235, 305-319) and keep all-zero weights."""
    rng = np.random.default_rng(rows + 7 * E)
    p = orc.softmax_rows(rng.standard_normal((rows, E)).astype(np.float32))
    valid = (rng.random(rows) < 0.7).astype(np.uint8)
    valid[0] = 0
    w, sel = orc.topk_mask(p, k, valid)
    idx = np.flatnonzero(valid)
    w_v, sel_v = orc.topk_mask(p[idx], k)
    np.testing.assert_array_equal(w[idx], w_v)
    np.testing.assert_array_equal(sel[idx], sel_v)
    assert np.all(w[valid == 0] == 0.0) and np.all(sel[valid == 0] == -1)
    counts, offsets, perm = orc.moe_dispatch_sel(sel, E)
    c_v, o_v, p_v = orc.moe_dispatch(w_v, k)
    np.testing.assert_array_equal(counts, c_v)
    np.testing.assert_array_equal(offsets, o_v)
    np.testing.assert_array_equal(perm[:offsets[-1]], idx[p_v])
    assert np.all(perm[offsets[-1]:] == -1) and offsets[-1] == len(idx) * k


def test_dispatch_of_selection_matches_dispatch_of_weights(orc):
    rng = np.random.default_rng(29)
    p = orc.softmax_rows(rng.standard_normal((257, 8)).astype(np.float32))
    w, sel = orc.topk_mask(p, 2)
    for a, b in zip(orc.moe_dispatch_sel(sel, 8), orc.moe_dispatch(w, 2)):
        np.testing.assert_array_equal(a, b)


def test_expert_loads(orc):
    """expert_loads (src/jamba.cpp:8299-8307): per-expert sums over the valid rows in
    ascending order; they sum to the number of valid rows (each renormalised row sums to
    1) and match a float64 column sum."""
    rng = np.random.default_rng(30)
    rows, E, k = 1000, 8, 2
    p = orc.softmax_rows(rng.standard_normal((rows, E)).astype(np.float32))
    valid = (rng.random(rows) < 0.8).astype(np.uint8)
    w, _ = orc.topk_mask(p, k, valid)
    loads = orc.expert_loads(w, valid)
    want = w[valid == 1].astype(np.float64).sum(axis=0)
    np.testing.assert_allclose(loads, want, rtol=1e-5)
    assert abs(float(loads.astype(np.float64).sum()) - int(valid.sum())) < 1e-2
    # in order: the running float sum, row by row
    run = np.zeros(E, np.float32)
    for r in range(rows):
        if valid[r]:
            run = (run + w[r]).astype(np.float32)
    np.testing.assert_array_equal(loads, run)
    # padding rows hold zero weights, so summing them too changes nothing
    np.testing.assert_array_equal(orc.expert_loads(w), loads)
