"""Pins the BitLinear part of the CPU oracle (CPU only).

Each check is chosen so a plausible restatement mistake fails it: the golden
vectors come from the reference's own compiled quantizer (oracle/_ref), the
integer GEMM is checked against an independent int64 product, and the
closed-form oracles are the reference's own test formulas
(OXN/nsos/tests/gpu/test_gpu_decode_runtime.cpp:54-75,
OXN/nsos/benchmarks/bench_decode_gemv.cpp:40-74).
"""
import hashlib
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def _golden():
    path = os.path.join(GOLDEN, "quant_ref.npz")
    want = open(os.path.join(GOLDEN, "MANIFEST.sha256")).read().split()[0]
    assert hashlib.sha256(open(path, "rb").read()).hexdigest() == want
    return np.load(path, allow_pickle=False)


def test_quantize_matches_reference_golden(orc):
    g = _golden()
    names = sorted({k.split("__")[0] for k in g.files if not k.startswith("rowsum")})
    assert names
    for name in names:
        x = g[f"{name}__x"]
        for bits in (2, 4, 8):
            q, s = orc.quantize_act(x, bits)
            want = np.clip(g[f"{name}__b{bits}__codes"], -127, 127).astype(np.int8)
            np.testing.assert_array_equal(q, want, err_msg=f"{name} bits={bits}")
            np.testing.assert_array_equal(s, g[f"{name}__b{bits}__scales"])


def test_quantize_rounding_rule_body_even_tail_away(orc):
    # x*s == x exactly when max|x| == 127 (s = 127/(127+1e-8f) rounds to 1.0f)
    x = np.zeros((1, 11), np.float32)
    x[0, 0] = 127.0
    x[0, 1:4] = [0.5, 1.5, 2.5]       # body (first 8): ties to even -> 0, 2, 2
    x[0, 8:11] = [0.5, 2.5, -0.5]     # tail (K%8 = 3): half away -> 1, 3, -1
    q, s = orc.quantize_act(x, 8)
    assert s[0] == np.float32(1.0)
    assert list(q[0, 1:4]) == [0, 2, 2]
    assert list(q[0, 8:11]) == [1, 3, -1]


@pytest.mark.skipif(not os.path.exists(os.path.join(os.path.dirname(__file__), "..", "oracle",
                                                     "_ref", "libnsos_ref.so")),
                    reason="oracle/_ref is built only where the reference is mounted")
def test_quantize_matches_reference_build_random(orc):
    rng = np.random.default_rng(7)
    for (m, k) in [(4, 8), (3, 17), (8, 2048), (2, 4093)]:
        x = (rng.standard_normal((m, k)) * rng.uniform(0.01, 50)).astype(np.float32)
        for bits in (2, 3, 8):
            codes, scales = orc.ref_quantize_rows(x, bits)
            q, s = orc.quantize_act(x, bits)
            np.testing.assert_array_equal(q, np.clip(codes, -127, 127).astype(np.int8))
            np.testing.assert_array_equal(s, scales)


def test_row_sums_match_reference_golden(orc):
    g = _golden()
    np.testing.assert_array_equal(orc.row_sums(g["rowsum__w"]), g["rowsum__sums"])


def test_act_scale_is_separate_division(orc):
    x = np.array([[0.3, -0.7, 0.1, 0.2, 0.5, -0.1, 0.0, 0.69]], np.float32)
    _, s = orc.quantize_act(x, 8)
    m = np.float32(0.7) + np.float32(1e-8)
    assert s[0] == np.float32(m / np.float32(127.0))
    assert orc.q_max(2) == 1.0 and orc.q_max(4) == 7.0 and orc.q_max(8) == 127.0


def test_pack_layout_closed_form(orc):
    # value -1 -> 0, 0 -> 1, +1 -> 2, element j of each group of four at bits 2j
    codes = np.array([-1, 0, 1, 1, 0, 0, -1, 1, 1], np.int8)
    packed = orc.pack_codes(codes)
    assert packed.tolist() == [0b10_10_01_00, 0b10_00_01_01, 0b10]
    np.testing.assert_array_equal(orc.unpack_codes(packed, codes.size), codes)


def test_unpack_reserved_code_is_zero_and_detected(orc):
    packed = np.array([0b11_10_01_00], np.uint8)
    assert orc.unpack_codes(packed, 4).tolist() == [-1, 0, 1, 0]
    assert orc.find_reserved_code(packed, 4) == 3
    assert orc.find_reserved_code(np.array([0b10_10_01_00], np.uint8), 4) == -1


def test_pack_round_trip_random(orc):
    rng = np.random.default_rng(1)
    codes = rng.integers(-1, 2, size=4099).astype(np.int8)
    np.testing.assert_array_equal(orc.unpack_codes(orc.pack_codes(codes), codes.size), codes)


def test_absmean_and_ternary_rule(orc):
    rng = np.random.default_rng(2)
    w = rng.standard_normal((37, 64)).astype(np.float32)
    want = np.float32(np.abs(w.astype(np.float64)).sum() / w.size)
    assert orc.absmean(w) == want
    ws = orc.weight_scale(w)
    assert ws == np.float32(want + np.float32(1e-8))
    codes = orc.ternary_codes(w, ws)
    thr = np.float32(ws + np.float32(1e-8))
    v = (w / thr).astype(np.float32)
    assert np.all(codes[v > 0.5] == 1) and np.all(codes[v < -0.5] == -1)
    assert np.all(codes[np.abs(v) <= 0.5] == 0)
    # a weight sitting exactly on the threshold stays 0 (strict inequality)
    w2 = np.array([[1.0, -1.0, 0.5, -0.5]], np.float32)
    ws2 = orc.weight_scale(w2)
    edge = np.float32(0.5) * np.float32(ws2 + np.float32(1e-8))
    w3 = np.array([[1.0, -1.0, edge, -edge]], np.float32)
    c3 = orc.ternary_codes(w3, ws2)
    assert c3[0, 0] == 1 and c3[0, 1] == -1


def test_gemm_i8_against_int64_product(orc):
    rng = np.random.default_rng(3)
    for (m, k, n) in [(1, 16, 5), (7, 48, 33), (16, 768, 64)]:
        q = rng.integers(-127, 128, size=(m, k)).astype(np.int8)
        w = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
        want = q.astype(np.int64) @ w.astype(np.int64).T
        np.testing.assert_array_equal(orc.gemm_i8(q, w), want.astype(np.int32))


def test_gemm_i8_extreme_magnitudes(orc):
    k = 4096
    q = np.full((2, k), 127, np.int8)
    q[1] = -127
    w = np.ones((3, k), np.int8)
    w[1] = -1
    w[2, ::2] = 0
    acc = orc.gemm_i8(q, w)
    assert acc.tolist() == [[127 * k, -127 * k, 127 * k // 2], [-127 * k, 127 * k, -127 * k // 2]]


def _decode_runtime_pattern(k, n, freq=.071):
    """Inputs of OXN/nsos/tests/gpu/test_gpu_decode_runtime.cpp:42-65."""
    x = np.sin(np.arange(1, k + 1, dtype=np.float32) * np.float32(freq)).astype(np.float32) * np.float32(.4)
    words = np.zeros(n * k // 16, np.uint32)
    for row in range(n):
        for kb in range(k // 16):
            word = 0
            for bit in range(16):
                word |= ((row + kb * 16 + bit) % 3) << (bit * 2)
            words[row * (k // 16) + kb] = word
    mag = (np.sin(np.arange(1, n + 1, dtype=np.float32) * np.float32(.12)) * np.float32(.4)).astype(np.float32)
    bias = (np.sin(np.arange(1, n + 1, dtype=np.float32) * np.float32(.1)) * np.float32(.4)).astype(np.float32)
    return x.astype(np.float32), words, mag, bias


@pytest.mark.parametrize("k,n", [(16, 3), (48, 17), (512, 33), (1024, 17)])
@pytest.mark.parametrize("bits", [2, 4, 8])
def test_decode_runtime_closed_form(orc, k, n, bits):
    """The reference's closed-form GEMV oracle, 2e-5 abs + rel as in that test."""
    x, words, mag, bias = _decode_runtime_pattern(k, n)
    qmax = np.float32((1 << (bits - 1)) - 1)
    den = np.float32(np.abs(x).max() + np.float32(1e-8))
    codes = np.array([[(row + kk) % 3 - 1 for kk in range(k)] for row in range(n)], np.int64)
    qx = np.round((x * (qmax / den)).astype(np.float32)).astype(np.int64)
    sums = codes @ qx
    ref = ((sums.astype(np.float32) * np.float32(.3)) * (den / qmax)) * mag + bias
    y = orc.bitlinear_forward(x[None, :], words, .3, n, bits=bits, magnitude=mag, bias=bias)[0]
    np.testing.assert_allclose(y, ref.astype(np.float32), atol=2e-5, rtol=2e-5)


def test_bench_decode_gemv_lcg_oracle(orc):
    """OXN/nsos/benchmarks/bench_decode_gemv.cpp:40-74 (LCG seed 20260919)."""
    k, n = 1024, 64
    i = np.arange(k, dtype=np.float32)
    x = (np.sin(i * np.float32(.013)) + np.float32(.25) * np.cos(i * np.float32(.037))).astype(np.float32)
    words = np.zeros(n * k // 16, np.uint32)
    r = 20260919
    for wi in range(words.size):
        word = 0
        for j in range(16):
            r = (r * 1664525 + 1013904223) & 0xFFFFFFFF
            word |= ((r >> 16) % 3) << (2 * j)
        words[wi] = word
    mx = np.float32(np.abs(x).max())
    inv = np.float32((mx + np.float32(1e-8)) / np.float32(127))
    scale = np.float32(np.float32(127) / (mx + np.float32(1e-8)))
    quant = np.rint(np.clip((x * scale).astype(np.float32), -127, 127)).astype(np.int64)
    wcodes = orc.unpack_codes(words, n * k).reshape(n, k).astype(np.int64)
    expected = (wcodes @ quant).astype(np.float32) * inv
    y = orc.bitlinear_forward(x[None, :], words, 1.0, n, bits=8)[0]
    assert np.all(np.abs(y - expected) <= 1e-4 + 1e-5 * np.abs(expected))


def test_dequant_order_and_fused_affine(orc):
    acc = np.array([[12345, -7, 0]], np.int32)
    s = np.array([np.float32(0.0123)], np.float32)
    ws = np.float32(0.77)
    mag = np.array([1.5, 0.25, 2.0], np.float32)
    bias = np.array([0.1, -0.2, 0.3], np.float32)
    y = orc.dequant(acc, s, ws, mag, bias)
    comb = np.float32(s[0] * ws)
    for j in range(3):
        v = np.float32(np.float32(acc[0, j]) * comb)
        # fma(v, mag, bias) evaluated exactly in float64 then rounded once
        want = np.float32(np.float64(v) * np.float64(mag[j]) + np.float64(bias[j]))
        assert y[0, j] == want
    y2 = orc.dequant(acc, s, ws)
    np.testing.assert_array_equal(y2[0], (acc[0].astype(np.float32) * comb).astype(np.float32))


def test_rmsnorm_matches_float64_within_ulps(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((5, 1024)).astype(np.float32)
    y = orc.rmsnorm(x, 1e-6)
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(axis=1, keepdims=True) + 1e-6)
    np.testing.assert_allclose(y, ref, rtol=2e-6, atol=0)


def test_bitlinear_rms_peri_composes(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    w = rng.standard_normal((32, 64)).astype(np.float32)
    packed, ws, codes = orc.pack_weights(w)
    y, q, s, acc = orc.bitlinear_forward(x, packed, ws, 32, rms_input=True, want_intermediates=True)
    q2, s2 = orc.quantize_act(orc.rmsnorm(x, 1e-6), 8)
    np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(s, s2)
    np.testing.assert_array_equal(acc, orc.gemm_i8(q2, codes))
    np.testing.assert_array_equal(y, orc.dequant(acc, s, ws))
