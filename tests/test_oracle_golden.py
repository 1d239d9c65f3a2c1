"""Pins the oracle to the reference's own compiled operators (CPU only).

tests/golden/tensor_ref.npz and bitlinear_ref.npz were written by
tests/golden/gen_golden.py from oracle/_ref, a build of the reference's
Tensor / BitLinear sources with the reference's flags.  Integer outputs and
the elementwise / row-wise float operators are compared bit for bit; the
float matmuls (whose summation order belongs to the reference's matmul_nt)
within 1e-6 relative.  A plausible restatement mistake (an fma the reference
does not form, a tree instead of an in-order sum, a dropped 1e-8f, the
renormalisation at k == E) fails one of these."""
import hashlib
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _load(name):
    path = os.path.join(GOLDEN, name)
    digests = dict(reversed(line.split()) for line in open(os.path.join(GOLDEN,
                                                                        "MANIFEST.sha256")))
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == digests[name]
    return np.load(path, allow_pickle=False)


def _f(a):
    return a.astype(np.float32)


def _bits_equal(got, want, what):
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[0]}: " \
                          f"{got.ravel()[bad[0]]!r} vs {want.ravel()[bad[0]]!r}"


@pytest.fixture(scope="module")
def tg():
    return _load("tensor_ref.npz")


@pytest.fixture(scope="module")
def bg():
    return _load("bitlinear_ref.npz")


@pytest.mark.parametrize("k", [768, 1024, 2048, 4096, 1003, 17, 7, 3])
def test_rmsnorm_and_rms_peri_codes_bit_exact(orc, tg, k):
    x = _f(tg[f"rms_k{k}__x"])
    y = orc.rmsnorm(x, 1e-6)
    _bits_equal(y, tg[f"rms_k{k}__y"], f"rmsnorm K={k}")
    q, s = orc.quantize_act(y, 8)
    np.testing.assert_array_equal(q, tg[f"rms_k{k}__codes"])
    _bits_equal(s, tg[f"rms_k{k}__scales"], f"act_scale K={k}")


@pytest.mark.parametrize("name", ["softmax", "softmax64"])
def test_softmax_bit_exact(orc, tg, name):
    _bits_equal(orc.softmax_rows(_f(tg[f"{name}__x"])), tg[f"{name}__y"], name)


def test_topk_keeps_raw_softmax_at_k_equal_e(orc, tg):
    probs = tg["softmax64__y"]
    w, sel = orc.topk_mask(probs, 64)
    _bits_equal(w, probs, "k == E weights")
    assert all(sorted(r) == list(range(64)) for r in sel)
    w2, _ = orc.topk_mask(probs, 63)      # k < E does renormalise
    assert not np.array_equal(w2, probs)


def test_activations_bit_exact(orc, tg):
    x = _f(tg["act__x"])
    g = _f(tg["act__g"])
    _bits_equal(orc.silu_array(x), tg["act__silu"], "silu")
    _bits_equal(x * orc.silu_array(g), tg["act__silu_gate"], "silu_gate")
    _bits_equal(orc.squared_relu(x), tg["act__squared_relu"], "squared_relu")


@pytest.mark.parametrize("n", [1, 7, 1000, 4099])
def test_abs_mean_bit_exact(orc, tg, n):
    got = np.float32(orc.absmean(_f(tg[f"absmean_n{n}__w"])))
    assert got == tg[f"absmean_n{n}__m"][0]


@pytest.mark.parametrize("k", [1024, 61])
def test_rmsnorm_backward_bit_exact(orc, tg, k):
    x = _f(tg[f"rmsbwd_k{k}__x"])
    dx = orc.rmsnorm_backward(x, _f(tg[f"rmsbwd_k{k}__g"]), orc.rmsnorm(x))
    _bits_equal(dx, tg[f"rmsbwd_k{k}__dx"], f"rmsnorm_backward K={k}")


CASES = ["rms_mag_bias", "rms_mag", "exact", "exact_bias", "gate_rms_mag",
                                  "exact_wide_bias"]


def _case(bg, name):
    get = lambda key: _f(bg[f"{name}__{key}"]) if f"{name}__{key}" in bg.files else None
    return {k: get(k) for k in ("w", "x", "grad", "mag", "bias")}, name.startswith("exact")


@pytest.mark.parametrize("name", CASES)
def test_bitlinear_packed_forward_bit_exact(orc, bg, name):
    c, exact = _case(bg, name)
    packed, ws, _ = orc.pack_weights(c["w"])
    y = orc.bitlinear_forward(c["x"], packed, ws, c["w"].shape[0], 8, not exact, c["mag"],
                              c["bias"])
    _bits_equal(y, bg[f"{name}__y_packed"], f"{name} packed forward")


@pytest.mark.parametrize("name", CASES)
def test_bitlinear_float_path(orc, bg, name):
    c, exact = _case(bg, name)
    y = orc.linear_f32(c["x"], c["w"], not exact, c["mag"], c["bias"])
    want = bg[f"{name}__y_float"]
    np.testing.assert_allclose(y, want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


@pytest.mark.parametrize("name", CASES)
def test_bitlinear_ste_backward(orc, bg, name):
    c, exact = _case(bg, name)
    o = orc.bitlinear_ste_backward(c["x"], c["w"], c["grad"], not exact, c["mag"],
                                   c["bias"] is not None)
    for key in ("dx", "dW", "dmag", "dbias"):
        if f"{name}__{key}" not in bg.files:
            assert key not in o or key == "dmag" and c["mag"] is not None
            continue
        want = bg[f"{name}__{key}"]
        np.testing.assert_allclose(o[key], want, rtol=1e-6, atol=1e-6 * np.abs(want).max(),
                                   err_msg=f"{name} {key}")


def test_ste_backward_planted_mistakes_fail(orc, bg):
    """The comparison above is tight enough to see a dropped magnitude multiply or a
    missing RMSNorm backward."""
    c, _ = _case(bg, "rms_mag_bias")
    want = bg["rms_mag_bias__dx"]
    no_rms = orc.bitlinear_ste_backward(c["x"], c["w"], c["grad"], False, c["mag"], True)
    assert not np.allclose(no_rms["dx"], want, rtol=1e-6, atol=1e-6 * np.abs(want).max())
    no_mag = orc.bitlinear_ste_backward(c["x"], c["w"], c["grad"], True, None, True)
    assert not np.allclose(no_mag["dx"], want, rtol=1e-6, atol=1e-6 * np.abs(want).max())


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle",
                                                     "_ref", "libnsos_ref.so")),
                    reason="oracle/_ref is built only where the reference is mounted")
def test_oracle_matches_reference_build_random(orc):
    from oracle import ref
    rng = np.random.default_rng(99)
    for k in (512, 1536, 33, 7, 3, 1, 65, 2050):
        x = (rng.standard_normal((16, k)) * rng.uniform(0.1, 9)).astype(np.float32)
        _bits_equal(orc.rmsnorm(x), ref.rmsnorm(x), f"rmsnorm K={k}")
        g = rng.standard_normal((16, k)).astype(np.float32)
        xn = orc.rmsnorm(x)
        _bits_equal(orc.rmsnorm_backward(x, g, xn), ref.rmsnorm_backward(x, g, xn), "rms bwd")
    lg = rng.standard_normal((4096, 16)).astype(np.float32) * 3
    _bits_equal(orc.softmax_rows(lg), ref.softmax(lg), "softmax")
    w = (rng.standard_normal((96, 256)) * 0.05).astype(np.float32)
    x = rng.standard_normal((9, 256)).astype(np.float32)
    mag = rng.uniform(0.5, 1.5, 96).astype(np.float32)
    bias = rng.standard_normal(96).astype(np.float32)
    packed, ws, _ = orc.pack_weights(w)
    _bits_equal(orc.bitlinear_forward(x, packed, ws, 96, 8, True, mag, bias),
                ref.bitlinear_forward(w, x, True, False, mag, bias), "packed forward")


def _mamba2_chain(orc, g, out_rms=False, dt_bias=True):
    """The oracle's restatement of Mamba2SSD::forward on its packed faithful path
    (src/mamba2.cpp:2360-2681): x / z / out_proj exact-linear ternary, B / C / dt float
    linear (dt with its bias), causal conv + SiLU per channel group, the selective scan
    without a gate, then RMSNorm(y * SiLU(z)) * norm weight."""
    H, P, N, G = (int(v) for v in g["shape"])
    p = {k: _f(g[k]) for k in ("w_x", "w_z", "w_B", "w_C", "w_dt", "dt_bias", "w_out",
                               "conv_w", "conv_b", "a_log", "d_skip", "norm_w")}
    inner, gs, d = H * P, G * N, p["w_out"].shape[0]
    px, wsx, _ = orc.pack_weights(p["w_x"])
    pz, wsz, _ = orc.pack_weights(p["w_z"])
    po, wso, _ = orc.pack_weights(p["w_out"])
    cw, cb = p["conv_w"], p["conv_b"]
    outs = []
    for ub in _f(g["u"]):
        cu = np.array([0, ub.shape[0]], np.int32)
        xv = orc.bitlinear_forward(ub, px, wsx, inner, 8, False)
        z = orc.bitlinear_forward(ub, pz, wsz, inner, 8, False)
        Bv = orc.linear_f32(ub, p["w_B"])
        Cv = orc.linear_f32(ub, p["w_C"])
        dt = orc.linear_f32(ub, p["w_dt"], bias=p["dt_bias"] if dt_bias else None)
        xc = orc.conv1d_causal(xv, cw[:inner], cu, bias=cb[:inner])
        Bc = orc.conv1d_causal(Bv, cw[inner:inner + gs], cu, bias=cb[inner:inner + gs])
        Cc = orc.conv1d_causal(Cv, cw[inner + gs:], cu, bias=cb[inner + gs:])
        y, _ = orc.selective_scan(xc, dt, p["a_log"], Bc, Cc, p["d_skip"], None, cu, H, P, N, G,
                                  gate_silu=False)
        normed = orc.rmsnorm_gated(y, z, p["norm_w"], eps=1e-5)
        outs.append(orc.bitlinear_forward(normed, po, wso, d, 8, out_rms))
    return np.stack(outs)


def test_mamba2_chain_matches_reference_build(orc):
    """tests/golden/mamba2_ref.npz holds Mamba2SSD::forward from a reference build
    (two sequences of 19 tokens, d_model 64, 4 heads of 32, d_state 16, 2 groups, conv 4).
    The chain's float stages sum in another order than the reference's matmul / conv
    loops, so the bound is fp32-level (1e-5 of the output scale); an out_proj with
    RMS_PERI or a dt projection without its bias is far outside it."""
    g = _load("mamba2_ref.npz")
    want = g["out_packed"]
    tol = 1e-5 * np.abs(want).max()
    got = _mamba2_chain(orc, g)
    assert np.abs(got - want).max() <= tol, np.abs(got - want).max()
    assert np.abs(_mamba2_chain(orc, g, out_rms=True) - want).max() > 100 * tol
    assert np.abs(_mamba2_chain(orc, g, dt_bias=False) - want).max() > 100 * tol


def test_mamba2_chain_matches_reference_build_d_state_64(orc):
    """tests/golden/mamba2_n64_ref.npz: Mamba2SSD::forward from a reference build at the
    reference's default state width (d_state 64; d_model 128, 4 heads of 64, 2 groups,
    conv 4, two sequences of 41 tokens), with the same bound and planted mistakes."""
    g = _load("mamba2_n64_ref.npz")
    assert tuple(int(v) for v in g["shape"]) == (4, 64, 64, 2)
    want = g["out_packed"]
    tol = 1e-5 * np.abs(want).max()
    got = _mamba2_chain(orc, g)
    assert np.abs(got - want).max() <= tol, np.abs(got - want).max()
    assert np.abs(_mamba2_chain(orc, g, out_rms=True) - want).max() > 100 * tol
    assert np.abs(_mamba2_chain(orc, g, dt_bias=False) - want).max() > 100 * tol
