"""Selective scan, decode step and causal conv on the GPU against the CPU oracle.

Tolerance (fp32 I/O): |gpu - oracle| <= 1e-5 + 1e-4 * |oracle| elementwise, the
north-star bound; the oracle forms decay in double, the GPU as exp2 of a float
product, and the readout sums states in a different order.  bf16 I/O: the
oracle runs in fp32 on the same bf16-rounded inputs; outputs within 2e-2
relative of the output scale (atol 2e-2 * max|oracle| / 64 plus rtol 2e-2)."""
import numpy as np
import pytest
import torch

from reimagined_amd import ops

pytestmark = pytest.mark.gpu
RTOL, ATOL = 1e-4, 1e-5


def _inputs(rng, T, H, P, N, G, per_state=True):
    D = H * P
    return dict(
        x=rng.standard_normal((T, D)).astype(np.float32),
        dt=rng.normal(-2.0, 0.5, (T, H)).astype(np.float32),
        a_log=rng.standard_normal((H, N) if per_state else (H,)).astype(np.float32),
        B=(rng.standard_normal((T, G * N)) * 0.25).astype(np.float32),
        C=(rng.standard_normal((T, G * N)) * 0.25).astype(np.float32),
        D=rng.standard_normal(H).astype(np.float32),
        z=rng.standard_normal((T, D)).astype(np.float32),
    )


def _t(dev, a, dtype=torch.float32):
    """Device copy; floating arrays are cast to `dtype`, integer arrays keep their type."""
    if a is None:
        return None
    t = torch.from_numpy(np.ascontiguousarray(a))
    if t.is_floating_point():
        t = t.to(dtype)
    return t.to(dev)


def _cu(lengths):
    return np.concatenate([[0], np.cumsum(lengths)]).astype(np.int32)


def _run(dev, orc, inp, cu, H, P, N, G, gate=True, init=None, dtype=torch.float32):
    args = [_t(dev, inp[k], dtype) for k in ("x", "dt")]
    cu_t = _t(dev, cu)
    assert cu_t.dtype == torch.int32
    y, fin = ops.selective_scan_fwd(
        args[0], args[1], _t(dev, inp["a_log"]), _t(dev, inp["B"], dtype), _t(dev, inp["C"], dtype),
        _t(dev, inp["D"]), _t(dev, inp["z"], dtype) if gate else None, cu_t, H, P, N, G,
        initial_state=_t(dev, init))
    return y.float().cpu().numpy(), fin.cpu().numpy()


@pytest.mark.parametrize("H,P,N,G,per_state,lengths", [
    (768, 1, 16, 1, True, [512]),                 # BASELINE config 2 shape
    (128, 1, 16, 1, True, [5, 64, 1, 33, 100]),   # ragged, lengths not multiples of 4
    (2, 64, 16, 1, False, [40, 7]),               # reference faithful: per-head A, P = 64
    (64, 1, 8, 1, True, [17]),                    # N = 8
    (64, 1, 13, 1, True, [21, 6]),                # N = 13: 16-state lanes, 3 padded states
    (2, 64, 14, 1, False, [40, 7]),               # per-head A, 2 padded states
    (4, 32, 16, 2, False, [9, 30]),               # G = 2, one group per workgroup
    (32, 1, 4, 1, True, [9, 22]),                 # N = 4: one state per lane
    (16, 2, 16, 2, False, [18, 5]),               # 16 channels per group
    (64, 1, 32, 1, True, [37, 5]),                # N = 32 -> LDS-staged kernel
    (128, 1, 64, 2, True, [6, 19]),               # N = 64, G = 2 -> LDS-staged kernel
    (6, 1, 5, 1, True, [11, 3]),                  # D = 6, N = 5 -> generic kernel
    (6, 2, 4, 3, False, [8, 2, 5]),               # 4 channels per group -> generic kernel
])
def test_scan_matches_oracle(dev, orc, H, P, N, G, per_state, lengths):
    rng = np.random.default_rng(H * 31 + N)
    cu = _cu(lengths)
    inp = _inputs(rng, int(cu[-1]), H, P, N, G, per_state)
    y, fin = _run(dev, orc, inp, cu, H, P, N, G)
    wy, wfin = orc.selective_scan(inp["x"], inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                                  inp["z"], cu, H, P, N, G)
    np.testing.assert_allclose(y, wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("count,hi", [(40, 12), (1100, 3)])
def test_scan_many_sequences_with_empty_ones(dev, orc, count, hi):
    """Empty sequences (equal cu_seqlens entries) and more sequences than the in-kernel
    longest-first ordering covers (1100 > 64: the order pre-pass): every non-empty sequence
    still matches the oracle and an empty one's final state is its (zero) initial state."""
    rng = np.random.default_rng(count)
    H, P, N, G = 32, 1, 16, 1
    lengths = rng.integers(0, hi + 1, size=count)
    lengths[::7] = 0
    cu = _cu(lengths)
    inp = _inputs(rng, int(cu[-1]), H, P, N, G)
    y, fin = _run(dev, orc, inp, cu, H, P, N, G)
    wy, wfin = orc.selective_scan(inp["x"], inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                                  inp["z"], cu, H, P, N, G)
    np.testing.assert_allclose(y, wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)
    assert np.all(fin[lengths == 0] == 0.0)


def test_scan_long_sequence_chunk_edges(dev, orc):
    """Lengths around the 32-token staging chunk and the 4-token group (the pipelined readout
    flushes the last group after the loop)."""
    rng = np.random.default_rng(77)
    H, P, N, G = 64, 1, 16, 1
    cu = _cu([31, 32, 33, 1001, 2, 4, 96])
    inp = _inputs(rng, int(cu[-1]), H, P, N, G)
    y, fin = _run(dev, orc, inp, cu, H, P, N, G)
    wy, wfin = orc.selective_scan(inp["x"], inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                                  inp["z"], cu, H, P, N, G)
    np.testing.assert_allclose(y, wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)


def test_scan_initial_state_and_no_gate(dev, orc):
    rng = np.random.default_rng(4)
    H, P, N, G = 128, 1, 16, 1
    cu = _cu([20, 45, 3])
    inp = _inputs(rng, int(cu[-1]), H, P, N, G)
    init = rng.normal(0, 0.1, (3, H * P, N)).astype(np.float32)
    y, fin = _run(dev, orc, inp, cu, H, P, N, G, gate=False, init=init)
    wy, wfin = orc.selective_scan(inp["x"], inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                                  None, cu, H, P, N, G, initial_state=init, gate_silu=False)
    np.testing.assert_allclose(y, wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)


def test_scan_ragged_equals_per_sequence(dev, orc):
    """A packed batch gives each sequence exactly what it gets alone (no leakage)."""
    rng = np.random.default_rng(8)
    H, P, N, G = 64, 1, 16, 1
    lengths = [13, 1, 70]
    cu = _cu(lengths)
    inp = _inputs(rng, int(cu[-1]), H, P, N, G)
    y, fin = _run(dev, orc, inp, cu, H, P, N, G)
    for s, (a, b) in enumerate(zip(cu[:-1], cu[1:])):
        part = {k: (v[a:b] if v.ndim == 2 and v.shape[0] == cu[-1] else v) for k, v in inp.items()}
        ys, fs = _run(dev, orc, part, _cu([b - a]), H, P, N, G)
        np.testing.assert_array_equal(ys, y[a:b])
        np.testing.assert_array_equal(fs[0], fin[s])


def test_scan_bf16_io(dev, orc):
    rng = np.random.default_rng(12)
    H, P, N, G = 256, 1, 16, 1
    cu = _cu([100, 37, 256])
    inp = _inputs(rng, int(cu[-1]), H, P, N, G)
    rb = {k: (torch.from_numpy(v).to(torch.bfloat16).float().numpy() if k in
              ("x", "dt", "B", "C", "z") else v) for k, v in inp.items()}
    y, fin = _run(dev, orc, inp, cu, H, P, N, G, dtype=torch.bfloat16)
    wy, wfin = orc.selective_scan(rb["x"], rb["dt"], rb["a_log"], rb["B"], rb["C"], rb["D"],
                                  rb["z"], cu, H, P, N, G)
    scale = np.abs(wy).max()
    np.testing.assert_allclose(y, wy, rtol=2e-2, atol=2e-2 * scale / 64)
    np.testing.assert_allclose(fin, wfin, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("H,P,N,G,per_state", [(256, 1, 16, 1, True), (4, 64, 16, 1, False),
                                               (8, 3, 5, 2, True), (100, 1, 8, 1, True),
                                               (64, 2, 32, 2, True), (96, 1, 64, 1, True),
                                               (40, 1, 4, 1, True)])
def test_step_matches_oracle_and_prefill(dev, orc, H, P, N, G, per_state):
    rng = np.random.default_rng(21 + N)
    R = 33
    inp = _inputs(rng, R, H, P, N, G, per_state)
    st0 = rng.normal(0, 0.1, (R, H * P, N)).astype(np.float32)
    state = _t(dev, st0)
    y = ops.selective_scan_step(_t(dev, inp["x"]), _t(dev, inp["dt"]), _t(dev, inp["a_log"]),
                                _t(dev, inp["B"]), _t(dev, inp["C"]), _t(dev, inp["D"]),
                                _t(dev, inp["z"]), state, H, P, N, G)
    wy, wst = orc.scan_step(inp["x"], inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                            inp["z"], st0, H, P, N, G)
    np.testing.assert_allclose(y.cpu().numpy(), wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(state.cpu().numpy(), wst, rtol=RTOL, atol=ATOL)
    # step == one-token prefill from the same state (src/mamba2.cpp:2814-2818 relies on it)
    yp, fp = _run(dev, orc, inp, _cu([1] * R), H, P, N, G, init=st0)
    np.testing.assert_allclose(y.cpu().numpy(), yp, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(state.cpu().numpy(), fp, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("R,offset_bc", [(256, 0), (37, 0), (37, 1), (1, 0), (3, 1)])
def test_step_bf16_config5(dev, orc, R, offset_bc):
    """Config 5's decode step: bf16 x, dt, z, B, C against an fp32 state [R, 2048, 16]
    (R = 256 is the bench's launch; 37, 3 and 1 rows leave a partial row block; B and C one
    element off 8-byte alignment take the two-byte loads).  The oracle runs in fp32 on the same
    bf16-rounded inputs; y within the bf16 bound, the state within the fp32 bound."""
    rng = np.random.default_rng(500 + R + offset_bc)
    H, P, N, G = 2048, 1, 16, 1
    inp = _inputs(rng, R, H, P, N, G, True)
    rb = {k: (torch.from_numpy(v).to(torch.bfloat16).float().numpy()
              if k in ("x", "dt", "B", "C", "z") else v) for k, v in inp.items()}
    st0 = rng.normal(0, 0.1, (R, H * P, N)).astype(np.float32)
    state = _t(dev, st0)
    bf = lambda k: _t(dev, inp[k], torch.bfloat16)
    if offset_bc:
        # B and C as [R, N] views one element into a larger buffer
        def shifted(k):
            big = torch.zeros(R * N + 1, dtype=torch.bfloat16, device=dev)
            big[1:] = _t(dev, inp[k], torch.bfloat16).reshape(-1)
            return big[1:].view(R, N)
        Bt, Ct = shifted("B"), shifted("C")
    else:
        Bt, Ct = bf("B"), bf("C")
    y = ops.selective_scan_step(bf("x"), bf("dt"), _t(dev, inp["a_log"]), Bt, Ct,
                                _t(dev, inp["D"]), bf("z"), state, H, P, N, G)
    wy, wst = orc.scan_step(rb["x"], rb["dt"], rb["a_log"], rb["B"], rb["C"], rb["D"], rb["z"],
                            st0, H, P, N, G)
    scale = np.abs(wy).max()
    np.testing.assert_allclose(y.float().cpu().numpy(), wy, rtol=2e-2, atol=2e-2 * scale / 64)
    np.testing.assert_allclose(state.cpu().numpy(), wst, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("H,G", [(2048, 4), (96, 2), (2040, 3)])
def test_step_bf16_groups(dev, orc, H, G):
    """bf16 decode steps with several B / C groups (P = 1, N = 16, 37 rows): groups of 512 and
    of 48 channels take the per-wave staged B / C (a workgroup of 64 channels spans two
    groups of 48, each wave one), groups of 680 channels are not whole 16-channel waves and
    take per-lane loads (2040 channels also leave a partial workgroup)."""
    rng = np.random.default_rng(700 + H + G)
    R, P, N = 37, 1, 16
    inp = _inputs(rng, R, H, P, N, G, True)
    rb = {k: (torch.from_numpy(v).to(torch.bfloat16).float().numpy()
              if k in ("x", "dt", "B", "C", "z") else v) for k, v in inp.items()}
    st0 = rng.normal(0, 0.1, (R, H * P, N)).astype(np.float32)
    state = _t(dev, st0)
    bf = lambda k: _t(dev, inp[k], torch.bfloat16)
    y = ops.selective_scan_step(bf("x"), bf("dt"), _t(dev, inp["a_log"]), bf("B"), bf("C"),
                                _t(dev, inp["D"]), bf("z"), state, H, P, N, G)
    wy, wst = orc.scan_step(rb["x"], rb["dt"], rb["a_log"], rb["B"], rb["C"], rb["D"], rb["z"],
                            st0, H, P, N, G)
    scale = np.abs(wy).max()
    np.testing.assert_allclose(y.float().cpu().numpy(), wy, rtol=2e-2, atol=2e-2 * scale / 64)
    np.testing.assert_allclose(state.cpu().numpy(), wst, rtol=RTOL, atol=ATOL)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_conv1d_matches_oracle(dev, orc, dtype):
    rng = np.random.default_rng(2)
    C, W = 96, 4
    cu = _cu([1, 2, 3, 10, 40])
    T = int(cu[-1])
    wide = rng.standard_normal((T, 2 * C)).astype(np.float32)  # x is the first half of each row
    w = rng.standard_normal((C, W)).astype(np.float32) * 0.5
    b = rng.standard_normal(C).astype(np.float32)
    wt = _t(dev, wide, dtype)
    out = ops.conv1d_causal(wt[:, :C], _t(dev, w), _t(dev, cu), _t(dev, b), silu=True,
                            out_dtype=torch.float32)
    x = wt[:, :C].float().cpu().numpy()
    want = orc.conv1d_causal(np.ascontiguousarray(x), w, cu, bias=b, silu_act=True)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=RTOL, atol=ATOL)


def test_scan_rejects_float_cu_seqlens(dev):
    x = torch.zeros((4, 64), device=dev)
    with pytest.raises(ValueError):
        ops.selective_scan_fwd(x, torch.zeros((4, 64), device=dev), torch.zeros((64, 16), device=dev),
                               torch.zeros((4, 16), device=dev), torch.zeros((4, 16), device=dev),
                               torch.zeros(64, device=dev), None,
                               torch.tensor([0.0, 4.0], device=dev), 64, 1, 16, 1)


@pytest.mark.parametrize("dtype,lengths,H,N,W", [
    (torch.float32, [5, 64, 1, 33], 128, 16, 4),
    (torch.bfloat16, [200, 3, 77], 128, 16, 4),
    (torch.float32, [2, 31, 6], 48, 16, 3),      # 48 channels: 16-channel waves only
    (torch.float32, [1, 9, 40], 64, 8, 2),
    (torch.bfloat16, [9, 30], 64, 15, 4),        # N = 15: one padded state
    (torch.float32, [7, 50], 64, 16, 6),        # width 6 -> LDS-staged kernel
    (torch.float32, [3, 26], 64, 32, 4),        # N = 32 -> LDS-staged kernel
])
def test_conv_scan_fused_matches_oracle(dev, orc, dtype, lengths, H, N, W):
    """conv + bias + SiLU fused into the scan == oracle conv, then oracle scan."""
    rng = np.random.default_rng(len(lengths) + H + W)
    P, G = 1, 1
    cu = _cu(lengths)
    T = int(cu[-1])
    inp = _inputs(rng, T, H, P, N, G)
    wide = rng.standard_normal((T, 2 * H)).astype(np.float32)  # raw x = left half of each row
    w = (rng.standard_normal((H, W)) * 0.5).astype(np.float32)
    b = (rng.standard_normal(H) * 0.1).astype(np.float32)
    wt = _t(dev, wide, dtype)
    zt = _t(dev, inp["z"], dtype)
    y, fin = ops.conv_scan_fwd(wt[:, :H], _t(dev, w), _t(dev, b), _t(dev, inp["dt"], dtype),
                               _t(dev, inp["a_log"]), _t(dev, inp["B"], dtype),
                               _t(dev, inp["C"], dtype), _t(dev, inp["D"]), zt, _t(dev, cu),
                               H, P, N, G)
    rd = lambda a: torch.from_numpy(a).to(dtype).float().numpy()
    xr = np.ascontiguousarray(wt[:, :H].float().cpu().numpy())
    xc = orc.conv1d_causal(xr, w, cu, bias=b, silu_act=True)
    if dtype == torch.float32:
        wy, wfin = orc.selective_scan(xc, inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                                      inp["z"], cu, H, P, N, G)
        np.testing.assert_allclose(y.cpu().numpy(), wy, rtol=RTOL, atol=ATOL)
        np.testing.assert_allclose(fin.cpu().numpy(), wfin, rtol=RTOL, atol=ATOL)
    else:
        wy, wfin = orc.selective_scan(xc, rd(inp["dt"]), inp["a_log"], rd(inp["B"]), rd(inp["C"]),
                                      inp["D"], rd(inp["z"]), cu, H, P, N, G)
        scale = np.abs(wy).max()
        np.testing.assert_allclose(y.float().cpu().numpy(), wy, rtol=2e-2, atol=2e-2 * scale / 64)
        np.testing.assert_allclose(fin.cpu().numpy(), wfin, rtol=1e-4, atol=1e-5)


# ---- time-chunked scan and the order pre-pass (nsosx_scan_fwd_planned) ------------------

def _scan_args(dev, inp, cu, dtype, gate):
    return dict(dt=_t(dev, inp["dt"], dtype), a_log=_t(dev, inp["a_log"]),
                B=_t(dev, inp["B"], dtype), C=_t(dev, inp["C"], dtype), D=_t(dev, inp["D"]),
                z=_t(dev, inp["z"], dtype) if gate else None, cu_seqlens=_t(dev, cu))


@pytest.mark.parametrize("conv", [False, True])
@pytest.mark.parametrize("chunk", [4, 37, 64, 200])
@pytest.mark.parametrize("per_state,P,gate,init", [(True, 1, True, False), (False, 16, False, True)])
def test_chunked_scan_matches_oracle(dev, orc, conv, chunk, per_state, P, gate, init):
    """Chunk boundaries inside sequences (carried state and conv window), sequences shorter
    than a chunk, an empty sequence, a chunk length that divides nothing (37): against the
    oracle within the fp32 bound, and against the unchunked scan to 1e-5."""
    rng = np.random.default_rng(chunk * 7 + int(conv) + P)
    H = 64 // P
    N, G = 16, 1
    lengths = [300, 0, 7, 64, 129, 1]
    cu = _cu(lengths)
    T = int(cu[-1])
    inp = _inputs(rng, T, H, P, N, G, per_state)
    a = _scan_args(dev, inp, cu, torch.float32, gate)
    st0 = rng.normal(0, 0.1, (len(lengths), H * P, N)).astype(np.float32) if init else None
    if conv:
        w = (rng.standard_normal((H * P, 4)) * 0.5).astype(np.float32)
        b = (rng.standard_normal(H * P) * 0.1).astype(np.float32)
        run = lambda ck: ops.conv_scan_fwd(_t(dev, inp["x"]), _t(dev, w), _t(dev, b), a["dt"],
                                           a["a_log"], a["B"], a["C"], a["D"], a["z"],
                                           a["cu_seqlens"], H, P, N, G,
                                           initial_state=_t(dev, st0), chunk_tokens=ck)
        xc = orc.conv1d_causal(inp["x"], w, cu, bias=b, silu_act=True)
    else:
        run = lambda ck: ops.selective_scan_fwd(_t(dev, inp["x"]), a["dt"], a["a_log"], a["B"],
                                                a["C"], a["D"], a["z"], a["cu_seqlens"], H, P, N,
                                                G, initial_state=_t(dev, st0), chunk_tokens=ck)
        xc = inp["x"]
    y, fin = (v.cpu().numpy() for v in run(chunk))
    y0, fin0 = (v.cpu().numpy() for v in run(0))
    wy, wfin = orc.selective_scan(xc, inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                                  inp["z"] if gate else None, cu, H, P, N, G,
                                  initial_state=st0, gate_silu=gate)
    np.testing.assert_allclose(y, wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(y, y0, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(fin, fin0, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("D", [128, 2048])
def test_chunked_auto_long_prefill(dev, orc, D):
    """The bench's long prefill: one 32768-token bf16 sequence with the fused conv and the
    chunk length the library picks (chunk_tokens = -1).  At 128 channels against the oracle
    (fp32 on the bf16-rounded inputs: y within the bf16 bound, the final state within the fp32
    bound); at the bench's 2048 channels against the sequential scan (y to one bf16 rounding,
    the final state to 1e-5)."""
    rng = np.random.default_rng(3 + D)
    T, H, P, N, G = 32768, D, 1, 16, 1
    inp = _inputs(rng, T, H, P, N, G, True)
    rb = {k: (torch.from_numpy(v).to(torch.bfloat16).float().numpy()
              if k in ("x", "dt", "B", "C", "z") else v) for k, v in inp.items()}
    w = (rng.standard_normal((D, 4)) * 0.5).astype(np.float32)
    b = (rng.standard_normal(D) * 0.1).astype(np.float32)
    cu = _cu([T])
    bf = lambda k: _t(dev, inp[k], torch.bfloat16)
    run = lambda ck: ops.conv_scan_fwd(bf("x"), _t(dev, w), _t(dev, b), bf("dt"),
                                       _t(dev, inp["a_log"]), bf("B"), bf("C"), _t(dev, inp["D"]),
                                       bf("z"), _t(dev, cu), H, P, N, G, chunk_tokens=ck,
                                       want_final=True)
    y, fin = run(-1)
    y, fin = y.float().cpu().numpy(), fin.cpu().numpy()
    if D == 128:
        xc = orc.conv1d_causal(rb["x"], w, cu, bias=b, silu_act=True)
        wy, wfin = orc.selective_scan(xc, rb["dt"], rb["a_log"], rb["B"], rb["C"], rb["D"],
                                      rb["z"], cu, H, P, N, G, gate_silu=True)
        scale = np.abs(wy).max()
        np.testing.assert_allclose(y, wy, rtol=2e-2, atol=2e-2 * scale / 64)
        np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)
    else:
        y0, fin0 = run(0)
        y0, fin0 = y0.float().cpu().numpy(), fin0.cpu().numpy()
        np.testing.assert_allclose(y, y0, rtol=2 ** -7, atol=1e-6)
        np.testing.assert_allclose(fin, fin0, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("chunk", [4, 37, 200])
@pytest.mark.parametrize("N,per_state,conv_w", [(64, False, 4), (64, True, 0), (32, False, 7),
                                                 (32, True, 4), (40, False, 0)])
def test_chunked_scan_wide_state_matches_oracle(dev, orc, chunk, N, per_state, conv_w):
    """The time-chunked scan above d_state 16 (the LDS-staged form): the faithful Mamba-2
    block's one A per head at the reference's default d_state 64 (src/include/nsos_config.h
    mamba_d_state), d_state 32, an N that is not a multiple of 16 (40), a conv window of 7
    that crosses several 4-token chunk boundaries, two groups of 64 channels: against the
    oracle within the fp32 bound and against the unchunked scan to 1e-5, final states
    included."""
    rng = np.random.default_rng(chunk * 13 + N + int(per_state) + conv_w)
    H, P, G = 2, 64, 2
    lengths = [300, 0, 7, 64, 129, 1]
    cu = _cu(lengths)
    T = int(cu[-1])
    inp = _inputs(rng, T, H, P, N, G, per_state)
    a = _scan_args(dev, inp, cu, torch.float32, True)
    st0 = rng.normal(0, 0.1, (len(lengths), H * P, N)).astype(np.float32)
    if conv_w:
        w = (rng.standard_normal((H * P, conv_w)) * 0.5).astype(np.float32)
        b = (rng.standard_normal(H * P) * 0.1).astype(np.float32)
        run = lambda ck: ops.conv_scan_fwd(_t(dev, inp["x"]), _t(dev, w), _t(dev, b), a["dt"],
                                           a["a_log"], a["B"], a["C"], a["D"], a["z"],
                                           a["cu_seqlens"], H, P, N, G,
                                           initial_state=_t(dev, st0), chunk_tokens=ck)
        xc = orc.conv1d_causal(inp["x"], w, cu, bias=b, silu_act=True)
    else:
        run = lambda ck: ops.selective_scan_fwd(_t(dev, inp["x"]), a["dt"], a["a_log"], a["B"],
                                                a["C"], a["D"], a["z"], a["cu_seqlens"], H, P, N,
                                                G, initial_state=_t(dev, st0), chunk_tokens=ck)
        xc = inp["x"]
    y, fin = (v.cpu().numpy() for v in run(chunk))
    y0, fin0 = (v.cpu().numpy() for v in run(0))
    wy, wfin = orc.selective_scan(xc, inp["dt"], inp["a_log"], inp["B"], inp["C"], inp["D"],
                                  inp["z"], cu, H, P, N, G, initial_state=st0)
    np.testing.assert_allclose(y, wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(y, y0, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(fin, fin0, rtol=1e-5, atol=1e-6)


def test_chunked_scan_auto_long_prefill_d_state_64(dev, orc):
    """One 4096-token prefill of the faithful block's shape at d_state 64 (8 heads of 64,
    one A per head, bf16 I/O): the library chunks it by itself; bf16 outputs within the
    bf16 bound, fp32 final state within 1e-4."""
    rng = np.random.default_rng(102)
    H, P, N, G = 8, 64, 64, 1
    cu = _cu([4096])
    inp = _inputs(rng, 4096, H, P, N, G, per_state=False)
    rd = lambda v: torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    w = (rng.standard_normal((H * P, 4)) * 0.5).astype(np.float32)
    a = _scan_args(dev, inp, cu, torch.bfloat16, True)
    assert int(ops.lib().nsosx_scan_fwd_workspace(1, 4096, H, P, N, -1)) > \
        int(ops.lib().nsosx_scan_fwd_workspace(1, 4096, H, P, N, 0))   # auto picks chunking
    y, fin = ops.conv_scan_fwd(_t(dev, inp["x"], torch.bfloat16), _t(dev, w), None, a["dt"],
                               a["a_log"], a["B"], a["C"], a["D"], a["z"], a["cu_seqlens"],
                               H, P, N, G)
    xc = orc.conv1d_causal(rd(inp["x"]), w, cu, silu_act=True)
    wy, wfin = orc.selective_scan(xc, rd(inp["dt"]), inp["a_log"], rd(inp["B"]), rd(inp["C"]),
                                  inp["D"], rd(inp["z"]), cu, H, P, N, G)
    scale = np.abs(wy).max()
    np.testing.assert_allclose(y.float().cpu().numpy(), wy, rtol=2e-2, atol=2e-2 * scale / 64)
    np.testing.assert_allclose(fin.cpu().numpy(), wfin, rtol=1e-4, atol=1e-5)


def test_chunked_scan_auto_long_prefill_bf16(dev, orc):
    """One 4096-token sequence over 512 channels: too few waves unchunked, so the library
    chunks it by itself; bf16 I/O within the bf16 bound, fp32 final state within 1e-4."""
    rng = np.random.default_rng(101)
    H, P, N, G = 512, 1, 16, 1
    cu = _cu([4096])
    inp = _inputs(rng, 4096, H, P, N, G)
    rd = lambda v: torch.from_numpy(v).to(torch.bfloat16).float().numpy()
    w = (rng.standard_normal((H, 4)) * 0.5).astype(np.float32)
    a = _scan_args(dev, inp, cu, torch.bfloat16, True)
    assert int(ops.lib().nsosx_scan_fwd_workspace(1, 4096, H, P, N, -1)) > \
        int(ops.lib().nsosx_scan_fwd_workspace(1, 4096, H, P, N, 0))   # auto picks chunking
    y, fin = ops.conv_scan_fwd(_t(dev, inp["x"], torch.bfloat16), _t(dev, w), None, a["dt"],
                               a["a_log"], a["B"], a["C"], a["D"], a["z"], a["cu_seqlens"],
                               H, P, N, G)
    xc = orc.conv1d_causal(rd(inp["x"]), w, cu, silu_act=True)
    wy, wfin = orc.selective_scan(xc, rd(inp["dt"]), inp["a_log"], rd(inp["B"]), rd(inp["C"]),
                                  inp["D"], rd(inp["z"]), cu, H, P, N, G)
    scale = np.abs(wy).max()
    np.testing.assert_allclose(y.float().cpu().numpy(), wy, rtol=2e-2, atol=2e-2 * scale / 64)
    np.testing.assert_allclose(fin.cpu().numpy(), wfin, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("count", [300, 1024])
def test_order_prepass_many_short_sequences(dev, orc, count):
    """Hundreds of sequences of 32-64 tokens (a continuous-batching step): with 300 the planned
    entry ranks them once in a pre-pass, with 1024 it keeps dispatch order; ordering changes
    only the schedule, so its outputs equal the unplanned entry's bit for bit, and both match
    the oracle."""
    rng = np.random.default_rng(55 + count)
    H, P, N, G = 128, 1, 16, 1
    lengths = rng.integers(32, 65, size=count)
    cu = _cu(lengths)
    inp = _inputs(rng, int(cu[-1]), H, P, N, G)
    a = _scan_args(dev, inp, cu, torch.float32, True)
    x = _t(dev, inp["x"])
    outs = [ops.selective_scan_fwd(x, a["dt"], a["a_log"], a["B"], a["C"], a["D"], a["z"],
                                   a["cu_seqlens"], H, P, N, G, chunk_tokens=ck)
            for ck in (0, None)]
    (y, fin), (yl, finl) = ((u.cpu().numpy(), v.cpu().numpy()) for u, v in outs)
    np.testing.assert_array_equal(y, yl)
    np.testing.assert_array_equal(fin, finl)
    wy, wfin = orc.selective_scan(inp["x"], inp["dt"], inp["a_log"], inp["B"], inp["C"],
                                  inp["D"], inp["z"], cu, H, P, N, G)
    np.testing.assert_allclose(y, wy, rtol=RTOL, atol=ATOL)
    np.testing.assert_allclose(fin, wfin, rtol=RTOL, atol=ATOL)
