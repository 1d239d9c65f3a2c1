"""BitLinear on the GPU against the CPU oracle: activation codes, int32
accumulators and fp32 outputs bit-exact; bf16 outputs equal to the oracle's
fp32 value rounded to bf16.  Covers the reference's golden quantizer vectors,
ragged and tail shapes, the decode GEMV for M = 1..8 and the MFMA GEMM."""
import os

import numpy as np
import pytest
import torch

from reimagined_amd import ops

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "quant_ref.npz")


def _bf16_round(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(torch.bfloat16).float().numpy()


def _weights(rng, n, k):
    return rng.standard_normal((n, k)).astype(np.float32)


def test_quantize_matches_reference_golden(dev, orc):
    g = np.load(GOLDEN, allow_pickle=False)
    names = sorted({k.split("__")[0] for k in g.files if not k.startswith("rowsum")})
    for name in names:
        x = g[f"{name}__x"]
        xt = torch.from_numpy(x).to(dev)
        for bits in (2, 4, 8):
            q, s = ops.quantize_activations_bitnet(xt, bits)
            want = np.clip(g[f"{name}__b{bits}__codes"], -127, 127).astype(np.int8)
            np.testing.assert_array_equal(q.cpu().numpy(), want, err_msg=f"{name} b{bits}")
            np.testing.assert_array_equal(s.cpu().numpy(), g[f"{name}__b{bits}__scales"])


@pytest.mark.parametrize("m,k", [(1, 16), (5, 1003), (33, 768), (7, 4096), (3, 8200), (64, 2048),
                                 (1500, 1024), (1100, 1003), (1029, 512), (1030, 4096), (1027, 2048),
                                 (8195, 1024), (4100, 2048)])
@pytest.mark.parametrize("rms", [False, True])
def test_quantize_random_f32(dev, orc, m, k, rms):
    rng = np.random.default_rng(m * 1000 + k)
    x = (rng.standard_normal((m, k)) * rng.uniform(0.1, 30)).astype(np.float32)
    q, s = ops.quantize_activations_bitnet(torch.from_numpy(x).to(dev), 8, rms_input=rms)
    src = orc.rmsnorm(x, 1e-6) if rms else x
    wq, ws = orc.quantize_act(src, 8)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)


@pytest.mark.parametrize("rms", [False, True])
@pytest.mark.parametrize("m,k", [(37, 1024), (1200, 1024), (1201, 2048), (1029, 512), (1026, 4096),
                                 (32769, 1024), (16411, 1024), (8200, 2048), (40796, 2048)])
def test_quantize_bf16_input(dev, orc, rms, m, k):
    """bf16 rows; M > 1024 with K = 512 / 1024 / 2048 / 4096 takes the several-rows-per-wave
    kernel, including row counts that leave a wave with rows past M.  The RMS pass is the
    three-wave form below 512 groups of 64 rows and the one-wave tiled form from 32705 rows
    (40796 x 2048: the out_proj input of the config-4 layer)."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((m, k)) * rng.uniform(0.5, 8.0, (m, 1))).astype(np.float32)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    q, s = ops.quantize_activations_bitnet(xb.to(dev), 8, rms_input=rms)
    xf = xb.float().numpy()
    wq, ws = orc.quantize_act(orc.rmsnorm(xf, 1e-6) if rms else xf, 8)
    np.testing.assert_array_equal(q.cpu().numpy(), wq)
    np.testing.assert_array_equal(s.cpu().numpy(), ws)


def _gemm_case(dev, orc, m, n, k, path, mag=False, bias=False, seed=0):
    rng = np.random.default_rng(seed + m * 7 + n * 13 + k)
    w = _weights(rng, n, k)
    packed, ws, codes = orc.pack_weights(w)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q, s = orc.quantize_act(x, 8)
    mg = rng.uniform(0.5, 1.5, n).astype(np.float32) if mag else None
    bs = rng.standard_normal(n).astype(np.float32) if bias else None
    acc_want = orc.gemm_i8(q, codes)
    y_want = orc.dequant(acc_want, s, ws, mg, bs)
    t = lambda a: None if a is None else torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    y, acc = ops.ternary_gemm(t(q), t(s), pk, ws, n, t(mg), t(bs), torch.float32, want_acc=True,
                              path=path)
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_want)
    np.testing.assert_array_equal(y.cpu().numpy(), y_want)
    # f32 without the accumulators: the MFMA GEMM's staged row epilogue where the tile allows
    yf = ops.ternary_gemm(t(q), t(s), pk, ws, n, t(mg), t(bs), torch.float32, path=path)
    np.testing.assert_array_equal(yf.cpu().numpy(), y_want)
    yb = ops.ternary_gemm(t(q), t(s), pk, ws, n, t(mg), t(bs), torch.bfloat16, path=path)
    np.testing.assert_array_equal(yb.float().cpu().numpy(), _bf16_round(y_want))


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("n,k", [(768, 768), (130, 2048), (64, 48), (33, 4096), (40, 8192),
                                 (1000, 256), (300, 128), (9000, 2048), (70, 12288),
                                 (37, 1040)])
def test_gemv_bit_exact(dev, orc, m, n, k):
    _gemm_case(dev, orc, m, n, k, path=0, mag=(m % 2 == 0), bias=(m % 3 == 0))


@pytest.mark.parametrize("m,n,k", [(16, 768, 768), (1, 64, 64), (129, 257, 1040), (300, 520, 2048),
                                   (256, 512, 48), (77, 1024, 4096)])
def test_mfma_gemm_bit_exact(dev, orc, m, n, k):
    _gemm_case(dev, orc, m, n, k, path=1, mag=True, bias=(n % 2 == 0))


@pytest.mark.parametrize("m,n,k", [(1000, 700, 512), (129, 256, 256), (513, 1024, 384),
                                   (2000, 96, 1024)])
def test_mfma_gemm_more_shapes_bit_exact(dev, orc, m, n, k):
    """LDS-staged MFMA GEMM: edge tiles in n and m, the shortest ring (K = 256), odd stage counts."""
    _gemm_case(dev, orc, m, n, k, path=1, mag=(m % 2 == 0), bias=True)


@pytest.mark.parametrize("m", [2, 3, 5, 8, 16, 17, 32])
@pytest.mark.parametrize("n,k", [(768, 1024), (130, 2048), (9000, 1024), (37, 2048), (64, 4096),
                                 (1, 1024)])
def test_skinny_mfma_bit_exact(dev, orc, m, n, k):
    """Decode-batch MFMA path: edge tiles in n, one and two m tiles, every K it accepts."""
    if (m + 15) // 16 * k > 4096:
        pytest.skip("outside the skinny path's LDS budget (ceil(M/16) * K <= 4096)")
    _gemm_case(dev, orc, m, n, k, path=2, mag=(m % 2 == 1), bias=(n % 2 == 0))


@pytest.mark.parametrize("m,k", [(9, 1024), (12, 2048), (16, 2048), (14, 4096), (17, 2048),
                                 (24, 1024), (32, 2048)])
@pytest.mark.parametrize("ydt", [torch.bfloat16, torch.float32])
def test_skinny_runs_of_tiles_bit_exact(dev, orc, m, k, ydt):
    """9-16 token rows over a matrix wide enough that every wave takes runs of 4
    consecutive tiles with whole-line output stores (N = 140000: 8750 tiles, a partial last
    run), and 17-32 rows (two m tiles: bf16 outputs in runs of 2 tiles), on the reference
    words (path 2) and the MFMA layout: equal bit for bit to the MFMA GEMM (path 1) on the
    same inputs, and to the oracle's dequantized sums on sampled columns (first, last and
    the partial run's)."""
    rng = np.random.default_rng(m * 7 + k + (ydt == torch.float32))
    n = 140000
    words = torch.randint(-2**31, 2**31 - 1, (n * k // 16,), dtype=torch.int32, device=dev)
    words = (words ^ ((words & (words >> 1) & 0x55555555) << 1)).contiguous()  # no code 3
    q_np = rng.integers(-127, 128, size=(m, k)).astype(np.int8)
    s_np = rng.uniform(0.001, 0.02, m).astype(np.float32)
    mag_np = rng.uniform(0.5, 1.5, n).astype(np.float32)
    bias_np = rng.standard_normal(n).astype(np.float32)
    q, s = torch.from_numpy(q_np).to(dev), torch.from_numpy(s_np).to(dev)
    mag, bias = torch.from_numpy(mag_np).to(dev), torch.from_numpy(bias_np).to(dev)
    want = ops.ternary_gemm(q, s, words, 0.37, n, mag, bias, out_dtype=ydt, path=1)
    got = ops.ternary_gemm(q, s, words, 0.37, n, mag, bias, out_dtype=ydt, path=2)
    got_mf = ops.ternary_gemm_mfma(q, s, ops.pack_mfma_layout(words), 0.37, n, mag, bias,
                                   out_dtype=ydt)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    assert torch.equal(got_mf, want)
    cols = np.unique(np.concatenate([[0, 15, 16, n - 33, n - 1],
                                     rng.choice(n, 251, replace=False)]))
    w_np = words.cpu().numpy().view(np.uint32).reshape(n, k // 16)[cols]
    codes = orc.unpack_codes(np.ascontiguousarray(w_np), cols.size * k).reshape(cols.size, k)
    acc = orc.gemm_i8(q_np, codes)
    y = orc.dequant(acc, s_np, 0.37, mag_np[cols], bias_np[cols])
    g = got.float().cpu().numpy()[:, cols]
    if ydt == torch.bfloat16:
        y = _bf16_round(y)
    np.testing.assert_array_equal(g, y)


@pytest.mark.parametrize("m,k", [(4, 768), (4, 1040), (1, 1024), (33, 1024), (17, 4096)])
def test_skinny_rejects_unsupported_shapes(dev, m, k):
    q = torch.zeros((m, k), dtype=torch.int8, device=dev)
    s = torch.ones(m, dtype=torch.float32, device=dev)
    pk = torch.zeros(64 * k // 16, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError, match="skinny"):
        ops.ternary_gemm(q, s, pk, 1.0, 64, path=2)


def test_gemm_dispatch_and_extremes(dev, orc):
    # |acc| = 127 * K at the extremes: int32 accumulation must not saturate or wrap
    k, n = 4096, 64
    q = np.full((9, k), 127, np.int8)
    q[1::2] = -127
    codes = np.ones((n, k), np.int8)
    codes[1::2] = -1
    packed = orc.pack_codes(codes).view(np.uint32)
    s = np.ones(9, np.float32)
    for path in (0, 1, 2):
        m = {0: 8, 1: 9, 2: 9}[path]
        y, acc = ops.ternary_gemm(torch.from_numpy(q[:m]).to(dev), torch.from_numpy(s[:m]).to(dev),
                                  torch.from_numpy(packed.view(np.int32)).to(dev), 1.0, n,
                                  want_acc=True, path=path)
        np.testing.assert_array_equal(acc.cpu().numpy(), orc.gemm_i8(q[:m], codes))


def test_reserved_code_is_zero_and_detected(dev, orc):
    rng = np.random.default_rng(5)
    n, k = 32, 64
    codes = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
    packed = orc.pack_codes(codes).view(np.uint32).copy()
    packed[7] |= 0x3 << 10  # element 7*16 + 5 becomes code 3
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    assert ops.find_reserved_code(pk, n * k) == 7 * 16 + 5
    codes_ref = orc.unpack_codes(packed, n * k).reshape(n, k)
    q = rng.integers(-127, 128, size=(4, k)).astype(np.int8)
    s = np.ones(4, np.float32)
    _, acc = ops.ternary_gemm(torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), pk, 1.0,
                              n, want_acc=True, path=0)
    np.testing.assert_array_equal(acc.cpu().numpy(), orc.gemm_i8(q, codes_ref))
    clean = torch.from_numpy(orc.pack_codes(codes).view(np.int32)).to(dev)
    assert ops.find_reserved_code(clean, n * k) == -1


@pytest.mark.parametrize("m", [1, 16, 200])
@pytest.mark.parametrize("rms", [False, True])
def test_bitlinear_forward_end_to_end(dev, orc, m, rms):
    rng = np.random.default_rng(m)
    n, k = 768, 768
    w = _weights(rng, n, k)
    packed, ws, _ = orc.pack_weights(w)
    x = rng.standard_normal((m, k)).astype(np.float32)
    mg = rng.uniform(0.5, 1.5, n).astype(np.float32)
    bs = rng.standard_normal(n).astype(np.float32)
    want = orc.bitlinear_forward(x, packed, ws, n, bits=8, rms_input=rms, magnitude=mg, bias=bs)
    y = ops.bitnet_gemm_158bit_gpu(torch.from_numpy(x).to(dev),
                                   torch.from_numpy(packed.view(np.int32)).to(dev), ws, m, k, n, 8,
                                   torch.from_numpy(mg).to(dev), torch.from_numpy(bs).to(dev),
                                   rms_input=rms)
    np.testing.assert_array_equal(y.cpu().numpy(), want)


def test_grouped_gemv_matches_per_group(dev, orc):
    rng = np.random.default_rng(9)
    groups, m, k, n = 5, 3, 1024, 256
    entries, wants, qs, ss = [], [], [], []
    for g in range(groups):
        w = _weights(rng, n, k)
        packed, ws, codes = orc.pack_weights(w)
        x = rng.standard_normal((m, k)).astype(np.float32)
        q, s = orc.quantize_act(x, 8)
        bias = rng.standard_normal(n).astype(np.float32) if g % 2 else None
        wants.append(orc.dequant(orc.gemm_i8(q, codes), s, ws, None, bias))
        entries.append((torch.from_numpy(packed.view(np.int32)).to(dev), ws, k, n, None,
                        None if bias is None else torch.from_numpy(bias).to(dev)))
        qs.append(q)
        ss.append(s)
    views = ops.LinearViewArray(entries, dev)
    y = ops.grouped_gemv(views, torch.from_numpy(np.stack(qs)).to(dev),
                         torch.from_numpy(np.stack(ss)).to(dev), n, out_dtype=torch.float32)
    np.testing.assert_array_equal(y.cpu().numpy(), np.stack(wants))


@pytest.mark.parametrize("m", [1, 2, 3, 8])
def test_grouped_gemv_mixed_shapes(dev, orc, m):
    """Groups of different K and N in one launch: K = 1024 / 2048 with N % 4 == 0 take the
    skinny MFMA body for M >= 2, the others (K = 768, N = 130) the VALU GEMV body."""
    from reimagined_amd._lib import call
    rng = np.random.default_rng(90 + m)
    shapes = [(1024, 256), (2048, 520), (768, 128), (1024, 130), (2048, 64)]
    kmax, nmax = max(k for k, _ in shapes), max(n for _, n in shapes)
    qbuf = np.zeros((len(shapes), m * kmax), np.int8)
    sbuf = np.zeros((len(shapes), m), np.float32)
    entries, wants = [], []
    for g, (k, n) in enumerate(shapes):
        w = _weights(rng, n, k)
        packed, ws, codes = orc.pack_weights(w)
        q, s = orc.quantize_act(rng.standard_normal((m, k)).astype(np.float32), 8)
        bias = rng.standard_normal(n).astype(np.float32) if g % 2 else None
        wants.append(orc.dequant(orc.gemm_i8(q, codes), s, ws, None, bias))
        entries.append((torch.from_numpy(packed.view(np.int32)).to(dev), ws, k, n, None,
                        None if bias is None else torch.from_numpy(bias).to(dev)))
        qbuf[g, :m * k] = q.reshape(-1)
        sbuf[g] = s
    views = ops.LinearViewArray(entries, dev)
    qd, sd = torch.from_numpy(qbuf).to(dev), torch.from_numpy(sbuf).to(dev)
    for dt in (torch.float32, torch.bfloat16):
        y = torch.full((len(shapes), m * nmax), 7.0, dtype=dt, device=dev)
        call("nsosx_grouped_gemv", views.ptr, len(shapes), qd.data_ptr(), m * kmax, sd.data_ptr(),
             m, m, y.data_ptr(), m * nmax, 0 if dt == torch.float32 else 1, None)
        got = y.float().cpu().numpy()
        for g, (k, n) in enumerate(shapes):
            want = wants[g] if dt == torch.float32 else _bf16_round(wants[g])
            np.testing.assert_array_equal(got[g, :m * n].reshape(m, n), want)
            assert np.all(got[g, m * n:] == 7.0)  # nothing written past the group's rows


def test_rejects_bad_arguments(dev):
    q = torch.zeros((2, 24), dtype=torch.int8, device=dev)
    s = torch.ones(2, device=dev)
    pk = torch.zeros(6, dtype=torch.int32, device=dev)
    with pytest.raises(ValueError):
        ops.ternary_gemm(q, s, pk, 1.0, 4)  # K % 16 != 0
    q = torch.zeros((2, 32), dtype=torch.int8, device=dev)
    with pytest.raises(ValueError):
        ops.ternary_gemm(q, s, pk, 0.0, 4)  # weight_scale must be > 0
    with pytest.raises(ValueError):
        ops.ternary_gemm(q, s, pk, 1.0, 4, path=0, want_y=False)  # no output


def test_config3_full_size_sampled(dev, orc):
    """Config 3 at full size through the dispatching entry point: the 4096 x 2048 x 8192 prefill
    GEMM (bf16 out, the bench's launch) bit-exact on sampled rows, and the decode GEMV / skinny
    paths on the same 8192 x 2048 weights at M = 1, 2, 16 and 32 bit-exact in full."""
    from reimagined_amd import workloads
    c3 = workloads.config3()
    packed, ws, codes = orc.pack_weights(c3["w"])
    q, s = orc.quantize_act(c3["x"], 8)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    y = ops.ternary_gemm(t(q), t(s), pk, ws, 8192, None, None, torch.bfloat16)
    rng = np.random.default_rng(33)
    rows = np.unique(np.concatenate([rng.choice(4096, 48, replace=False), [0, 4095]]))
    y_want = orc.dequant(orc.gemm_i8(q[rows], codes), s[rows], ws, None, None)
    np.testing.assert_array_equal(y[t(rows)].float().cpu().numpy(), _bf16_round(y_want))
    for m in (1, 2, 16, 32):
        yd, acc = ops.ternary_gemm(t(q[:m]), t(s[:m]), pk, ws, 8192, None, None, torch.float32,
                                   want_acc=True)
        acc_want = orc.gemm_i8(q[:m], codes)
        np.testing.assert_array_equal(acc.cpu().numpy(), acc_want)
        np.testing.assert_array_equal(yd.cpu().numpy(), orc.dequant(acc_want, s[:m], ws, None, None))


@pytest.mark.parametrize("shift_y,shift_affine", [(0, 1), (1, 0), (4, 4)])
def test_gemm_epilogue_alignment(dev, orc, shift_y, shift_affine):
    """The MFMA GEMM's row-store epilogue needs 16-byte aligned output, magnitude and bias;
    outputs and affine vectors that start a few elements into their buffers take the
    accumulator-order stores instead, with the same bits (bf16 output, magnitude and bias)."""
    from reimagined_amd._lib import call
    from reimagined_amd.ops import _p, _stream
    rng = np.random.default_rng(71 + shift_y * 3 + shift_affine)
    m, n, k = 300, 768, 512
    w = _weights(rng, n, k)
    packed, ws, codes = orc.pack_weights(w)
    x = rng.standard_normal((m, k)).astype(np.float32)
    q, s = orc.quantize_act(x, 8)
    mg = rng.uniform(0.5, 1.5, n).astype(np.float32)
    bs = rng.standard_normal(n).astype(np.float32)
    y_want = _bf16_round(orc.dequant(orc.gemm_i8(q, codes), s, ws, mg, bs))
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    mg_buf = torch.zeros(n + shift_affine, dtype=torch.float32, device=dev)
    bs_buf = torch.zeros(n + shift_affine, dtype=torch.float32, device=dev)
    mg_buf[shift_affine:] = t(mg)
    bs_buf[shift_affine:] = t(bs)
    y_buf = torch.zeros(m * n + shift_y, dtype=torch.bfloat16, device=dev)
    y = y_buf[shift_y:].view(m, n)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    qd, sd = t(q), t(s)  # held until the kernel has run: a freed temporary is reused at once
    call("nsosx_ternary_gemm_path", _p(qd), _p(sd), _p(pk), ws, m, k, n,
         _p(mg_buf[shift_affine:]), _p(bs_buf[shift_affine:]), _p(y), 1, None, 1, _stream())
    np.testing.assert_array_equal(y.float().cpu().numpy(), y_want)


@pytest.mark.parametrize("n,k", [(6, 1000 // 16 * 16), (4096, 1024), (1, 16), (1023, 2048)])
def test_weight_row_sums_match_oracle(dev, orc, n, k):
    """compute_weight_row_sums on the device, from the packed words, against the oracle's
    int8 row sums (pinned by the reference build's golden rowsum__sums)."""
    rng = np.random.default_rng(n + k)
    codes = rng.integers(-1, 2, size=(n, k)).astype(np.int8)
    packed = orc.pack_codes(codes).view(np.uint32)
    got = ops.weight_row_sums(torch.from_numpy(packed.view(np.int32)).to(dev), n, k)
    np.testing.assert_array_equal(got.cpu().numpy(), orc.row_sums(codes))


def test_weight_row_sums_golden_and_reserved_code(dev, orc):
    g = np.load(GOLDEN, allow_pickle=False)
    w = g["rowsum__w"][:, :992]          # K % 16 == 0 prefix of the golden rows
    want = g["rowsum__w"][:, :992].astype(np.int32).sum(1)
    packed = orc.pack_codes(w).view(np.uint32)
    got = ops.weight_row_sums(torch.from_numpy(packed.view(np.int32)).to(dev), 6, 992)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    np.testing.assert_array_equal(orc.row_sums(w), want)
    # full golden rows through the oracle, which the reference build pinned
    np.testing.assert_array_equal(orc.row_sums(g["rowsum__w"]), g["rowsum__sums"])
    # the reserved code 3 decodes to 0 and adds nothing
    words = np.array([0xFFFFFFFF, 0x66666666, 0x00000000, 0xAAAAAAAA], np.uint32)
    got = ops.weight_row_sums(torch.from_numpy(words.view(np.int32)).to(dev), 4, 16)
    np.testing.assert_array_equal(got.cpu().numpy(), [0, 8, -16, 16])


@pytest.mark.parametrize("m,k,n", [(300, 1024, 700), (129, 384, 256), (1000, 512, 520),
                                   (4096, 2048, 8192), (1, 128, 16), (257, 2048, 1024),
                                   # decode batches: the skinny kernel on the MFMA layout
                                   (2, 1024, 700), (16, 2048, 520), (17, 2048, 1024),
                                   (32, 2048, 8192), (5, 4096, 66)])
@pytest.mark.parametrize("ydt,acc", [(torch.bfloat16, False), (torch.float32, True),
                                     (torch.float32, False)])
def test_gemm_mfma_layout_matches_reference_layout(dev, orc, m, k, n, ydt, acc):
    """The GEMM on repacked (MFMA-layout) weights -- the prefill MFMA GEMM, and the skinny
    decode kernel at 2 <= M <= 32 -- gives the reference-layout GEMM's outputs bit for bit,
    including words holding the reserved code 3 (decoded to 0 by both), edge tiles in M and N,
    magnitude and bias; the accumulators match the oracle."""
    rng = np.random.default_rng(m + k + n)
    words = torch.randint(-2**31, 2**31 - 1, (n * k // 16,), dtype=torch.int32, device=dev)
    q = torch.from_numpy(rng.integers(-127, 128, size=(m, k)).astype(np.int8)).to(dev)
    s = torch.from_numpy(rng.uniform(0.001, 0.02, m).astype(np.float32)).to(dev)
    mag = torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float32)).to(dev)
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(dev)
    mf = ops.pack_mfma_layout(words)
    for mg, b in ((None, None), (mag, bias)):
        want = ops.ternary_gemm(q, s, words, 0.37, n, mg, b, out_dtype=ydt, want_acc=acc, path=1)
        got = ops.ternary_gemm_mfma(q, s, mf, 0.37, n, mg, b, out_dtype=ydt, want_acc=acc)
        torch.cuda.synchronize()
        if acc:
            assert torch.equal(got[1], want[1])
            got, want = got[0], want[0]
        assert torch.equal(got, want)
    if acc and m * n <= 300 * 1024:
        codes = orc.unpack_codes(words.cpu().numpy().view(np.uint32), n * k).reshape(n, k)
        _, a = ops.ternary_gemm_mfma(q, s, mf, 0.37, n, want_acc=True)
        np.testing.assert_array_equal(a.cpu().numpy(), orc.gemm_i8(q.cpu().numpy(), codes))


@pytest.mark.parametrize("gather,sqrelu", [(True, True), (False, False)])
def test_grouped_gemm_mfma_matches_reference_layout(dev, gather, sqrelu):
    rng = np.random.default_rng(5 + gather)
    counts = [0, 1, 129, 0, 300, 64, 257]
    E, K, N = len(counts), 384, 520
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    slots = int(offsets[-1])
    rows = slots + 17
    q = torch.from_numpy(rng.integers(-127, 128, size=(rows, K)).astype(np.int8)).to(dev)
    s = torch.from_numpy(rng.uniform(0.001, 0.02, rows).astype(np.float32)).to(dev)
    perm = torch.from_numpy((rng.permutation(rows)[:slots] if gather else np.arange(slots))
                            .astype(np.int32)).to(dev)
    ref_e, mf_e = [], []
    for e in range(E):
        w = torch.randint(-2**31, 2**31 - 1, (N * K // 16,), dtype=torch.int32, device=dev)
        mg = torch.from_numpy(rng.uniform(0.5, 1.5, N).astype(np.float32)).to(dev)
        bs = torch.from_numpy(rng.standard_normal(N).astype(np.float32)).to(dev)
        ref_e.append((w, 0.1 + 0.01 * e, K, N, mg, bs))
        mf_e.append((ops.pack_mfma_layout(w), 0.1 + 0.01 * e, K, N, mg, bs))
    off = torch.from_numpy(offsets).to(dev)
    qq, ss = (q, s) if gather else (q[:slots], s[:slots])
    want = ops.grouped_ternary_gemm(ops.LinearViewArray(ref_e, dev), off, perm, qq, ss, N,
                                    max(counts), sqrelu, gather, torch.bfloat16)
    got = ops.grouped_ternary_gemm_mfma(ops.LinearViewArray(mf_e, dev), off, perm, qq, ss, N,
                                        slots, sqrelu, gather, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("m,k,dtype", [(16411, 1024, torch.bfloat16), (8200, 2048, torch.bfloat16),
                                       (8195, 1024, torch.float32), (4100, 2048, torch.float32),
                                       (8000, 1024, torch.bfloat16), (3001, 2048, torch.bfloat16),
                                       (1500, 1024, torch.float32), (1027, 2048, torch.float32)])
def test_rms_workspace_in_order_sum(dev, m, k, dtype):
    """The RMS_PERI row scale left in rms_workspace (the STE backward reads it) by the
    tiled and the producer / consumer RMS passes:
    1 / sqrt(mean + 1e-6) of the in-order float sum of the rounded squares
    (Tensor::rmsnorm, src/tensor.cpp:3455-3492); numpy's add.accumulate adds in order."""
    from reimagined_amd._lib import call
    from reimagined_amd.ops import _p, _dt, _stream
    rng = np.random.default_rng(m + k)
    x = (rng.standard_normal((m, k)) * rng.uniform(0.5, 8.0, (m, 1))).astype(np.float32)
    xt = torch.from_numpy(x).to(dtype)
    xf = xt.float().numpy()
    xd = xt.to(dev)
    q = torch.empty((m, k), dtype=torch.int8, device=dev)
    s = torch.empty(m, dtype=torch.float32, device=dev)
    rw = torch.empty(m, dtype=torch.float32, device=dev)
    call("nsosx_quantize_act_i8", _p(xd), _dt(xd), m, k, 8, 1, _p(q), _p(s), _p(rw), _stream())
    sq = (xf * xf).astype(np.float32)
    total = np.add.accumulate(sq, axis=1, dtype=np.float32)[:, -1]
    want = (np.float32(1.0) / np.sqrt(total / np.float32(k) + np.float32(1e-6))).astype(np.float32)
    np.testing.assert_array_equal(rw.cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_grouped_decode_projections_match_single_calls(dev, dtype):
    """One input row through packed and float views in one launch
    (GpuProjectionGroup::forward, src/gpu_projection_group.cpp:12-49): each packed view
    equals nsosx_bitlinear_forward at M = 1 and each float view nsosx_linear_f32 at M = 1,
    bit for bit (RMS_PERI, magnitude, bias, 4-bit activations, a view over the first 512
    inputs); a view outside the supported shapes writes nothing."""
    rng = np.random.default_rng(44)
    K = 1024
    x = torch.from_numpy(rng.standard_normal((1, K)).astype(np.float32) * 3).to(dtype).to(dev)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)
    specs = [("packed", 2048, K, 8, False, False, False), ("packed", 1024, K, 8, True, True, True),
             ("float", 64, K, 0, False, False, True), ("float", 8, K, 0, True, True, False),
             ("packed", 768, K, 4, False, True, False), ("packed", 256, 512, 8, True, False, True),
             ("packed", 16, 1000, 8, False, False, False)]
    entries, refs = [], []
    for kind, n, k, bits, rms, mag, bias in specs:
        w = rng.standard_normal((n, k)).astype(np.float32)
        m_ = t(rng.uniform(0.5, 1.5, n)) if mag else None
        b_ = t(rng.standard_normal(n)) if bias else None
        e = {"inputs": k, "outputs": n, "rms_input": rms, "magnitude": m_, "bias": b_}
        if kind == "packed":
            packed, ws = ops.pack_ternary(w) if k % 16 == 0 else (np.zeros(n * k // 16 + 1, np.uint32), 1.0)
            pk = torch.from_numpy(packed.view(np.int32)).to(dev)
            e.update(packed=pk, weight_scale=ws, bits=bits)
            want = (ops.bitnet_gemm_158bit_gpu(x[:, :k].contiguous(), pk, ws, 1, k, n, bits, m_, b_,
                                               rms_input=rms) if k % 64 == 0 else None)
        else:
            wt = t(w)
            e.update(weight=wt)
            want = ops.linear_f32(x[:, :k].contiguous(), wt, rms_input=rms, magnitude=m_, bias=b_)
        entries.append(e)
        refs.append(want)
    views = ops.DecodeViewArray(entries, dev)
    out = torch.full((len(specs), views.max_outputs), 7.0, device=dev)
    ops.grouped_decode_projections(views, x[0], out=out)
    got = out.cpu().numpy()
    for i, ((kind, n, *_), want) in enumerate(zip(specs, refs)):
        if want is None:
            assert (got[i] == 7.0).all()
        else:
            np.testing.assert_array_equal(got[i, :n], want.float().cpu().numpy()[0])


@pytest.mark.parametrize("m,k", [(2, 1024), (7, 2048), (16, 1024), (32, 2048), (300, 1024)])
def test_layer_bitlinear_decode_batches_bit_exact(dev, orc, m, k):
    """layers.BitLinear at decode-batch sizes runs the skinny MFMA kernel on its MFMA-layout
    copy (and the prefill GEMM above 128 rows): RMS_PERI, magnitude and bias included, the
    outputs equal the reference BitLinear::forward restatement bit for bit."""
    from reimagined_amd.layers import BitLinear
    rng = np.random.default_rng(m * 31 + k)
    n = 520
    w = _weights(rng, n, k)
    mg = rng.uniform(0.5, 1.5, n).astype(np.float32)
    bs = rng.standard_normal(n).astype(np.float32)
    lin = BitLinear(w, dev, rms_input=True, magnitude=torch.from_numpy(mg).to(dev),
                    bias=torch.from_numpy(bs).to(dev))
    assert lin.packed_mfma is not None
    packed, ws, _ = orc.pack_weights(w)
    x = rng.standard_normal((m, k)).astype(np.float32)
    want = orc.bitlinear_forward(x, packed, ws, n, bits=8, rms_input=True, magnitude=mg, bias=bs)
    y = lin.forward(torch.from_numpy(x).to(dev), out_dtype=torch.float32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(y.cpu().numpy(), want)
