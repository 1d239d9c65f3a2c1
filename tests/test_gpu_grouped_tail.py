"""The grouped MFMA GEMM's split-K tail (nsosx_grouped_ternary_gemm_mfma_ws).

A launch whose last round of 256 x 128 tiles would leave three quarters of the resident
workgroups idle, with K of at least 16 stages (2048), splits those tiles along K and adds the
int32 partial sums in a second launch.  Integer sums are exact, so every case is bit-exact
against the whole-tile entry (nsosx_grouped_ternary_gemm_mfma) on the same inputs: the routed
config-5 down GEMM (an 8-way split of its tail), 4-way splits with magnitude and bias (f32 out,
also checked against the oracle) and with gathered rows, squared ReLU and bf16 out, and
launches left whole (the up GEMM's K = 1024 tiles are too short to split)."""
import numpy as np
import pytest
import torch

from reimagined_amd import ops

pytestmark = pytest.mark.gpu

ROUTED = [2109, 2004, 2063, 2018, 1998, 2108, 2029, 2055]  # config-5 routing, 16384 slots


def _random_views(dev, E, K, N, seed):
    """E random ternary [N, K] matrices in the MFMA layout, generated on the device."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    entries = []
    for _ in range(E):
        p = torch.randint(-2**31, 2**31 - 1, (N * K // 16,), dtype=torch.int32, device=dev,
                          generator=g)
        p = (p ^ ((p & (p >> 1) & 0x55555555) << 1)).contiguous()  # no reserved code 3
        entries.append((ops.pack_mfma_layout(p), 0.37, K, N, None, None))
    return ops.LinearViewArray(entries, dev)


def _ab(dev, views, counts, K, N, gather, sqrelu, out_dtype, seed):
    rng = np.random.default_rng(seed)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    slots = int(offsets[-1])
    rows = slots // 2 + 5 if gather else slots
    q = torch.from_numpy(rng.integers(-127, 128, size=(rows, K), dtype=np.int8)).to(dev)
    s = torch.from_numpy(rng.uniform(0.001, 0.02, rows).astype(np.float32)).to(dev)
    perm = (torch.from_numpy(rng.integers(0, rows, slots).astype(np.int32)).to(dev)
            if gather else None)
    offd = torch.from_numpy(offsets).to(dev)
    ws = torch.empty(ops.grouped_mfma_workspace_bytes(), dtype=torch.uint8, device=dev)
    want = ops.grouped_ternary_gemm_mfma(views, offd, perm, q, s, N, slots, sqrelu, gather,
                                         out_dtype)
    for _ in range(2):  # the workspace is reused: a second call must not see the first's sums
        got = ops.grouped_ternary_gemm_mfma(views, offd, perm, q, s, N, slots, sqrelu, gather,
                                            out_dtype, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(got, want)
    return q, s, perm, offsets, got


def test_split_tail_down_routed(dev):
    K, N = 4096, 1024  # 528 tiles on 512 resident workgroups: 16 tail tiles split 8 ways
    views = _random_views(dev, 8, K, N, 5)
    _ab(dev, views, ROUTED, K, N, False, False, torch.float32, 1)


def test_up_routed_left_whole(dev):
    K, N = 1024, 4096  # 2112 tiles, a 64-tile tail of 8-stage tiles: not split
    views = _random_views(dev, 8, K, N, 6)
    _ab(dev, views, ROUTED, K, N, True, True, torch.bfloat16, 2)


def test_split_tail_sqrelu_bf16(dev):
    K, N = 2048, 1024  # 544 tiles: the 32-tile tail split 4 ways, squared ReLU, bf16 out
    views = _random_views(dev, 8, K, N, 8)
    _ab(dev, views, [2098] * 8, K, N, True, True, torch.bfloat16, 5)


@pytest.mark.parametrize("counts,K,N", [([2048] * 8, 4096, 1024),          # whole rounds
                                        ([0, 1, 129, 0, 300, 64, 257], 384, 520),  # one round
                                        ([3000, 0, 2500], 2048, 768)])
def test_no_split_matches(dev, counts, K, N):
    views = _random_views(dev, len(counts), K, N, 7 + K)
    _ab(dev, views, counts, K, N, False, False, torch.float32, 3)


def test_split_tail_against_oracle(dev, orc):
    """K = 2048 (16 k-stages), 8 experts of 2098 rows: 544 tiles, the 32-tile tail split 4 ways
    (4 k-stages each), magnitude and bias, gathered rows, f32 out.  Bit-exact against the
    whole-tile entry, and each expert's last 50 rows (its partial tile, split) against the
    oracle's dequantized product."""
    E, K, N = 8, 2048, 1024
    rng = np.random.default_rng(21)
    entries, codes, wss, mags, biases = [], [], [], [], []
    for _ in range(E):
        pk, wsc, cd = orc.pack_weights(rng.standard_normal((N, K)).astype(np.float32))
        mg = rng.uniform(0.5, 1.5, N).astype(np.float32)
        bs = rng.standard_normal(N).astype(np.float32)
        words = torch.from_numpy(pk.view(np.int32)).to(dev)
        entries.append((ops.pack_mfma_layout(words), wsc, K, N, torch.from_numpy(mg).to(dev),
                        torch.from_numpy(bs).to(dev)))
        codes.append(cd); wss.append(wsc); mags.append(mg); biases.append(bs)
    views = ops.LinearViewArray(entries, dev)
    q, s, perm, offsets, got = _ab(dev, views, [2098] * E, K, N, True, False, torch.float32, 4)
    qn, sn, pn, y = q.cpu().numpy(), s.cpu().numpy(), perm.cpu().numpy(), got.cpu().numpy()
    for e in range(E):
        lo, hi = int(offsets[e + 1]) - 50, int(offsets[e + 1])
        src = pn[lo:hi]
        want = orc.dequant(orc.gemm_i8(qn[src], codes[e]), sn[src], wss[e], mags[e], biases[e])
        np.testing.assert_array_equal(y[lo:hi], want, err_msg=f"expert {e}")


def test_workspace_checked(dev):
    from reimagined_amd._lib import lib
    L = lib()
    need = ops.grouped_mfma_workspace_bytes()
    assert need > 0 and need % (128 * 1024) == 0
    views = _random_views(dev, 2, 128, 256, 9)
    offd = torch.tensor([0, 10, 20], dtype=torch.int32, device=dev)
    q = torch.zeros((20, 128), dtype=torch.int8, device=dev)
    s = torch.ones(20, dtype=torch.float32, device=dev)
    y = torch.empty((20, 256), dtype=torch.float32, device=dev)
    small = torch.empty(need - 16, dtype=torch.uint8, device=dev)
    rc = L.nsosx_grouped_ternary_gemm_mfma_ws(views.ptr, 2, offd.data_ptr(), None, 0,
                                              q.data_ptr(), s.data_ptr(), 128, 256, 20, 0,
                                              y.data_ptr(), 0, small.data_ptr(), need - 16, None)
    assert rc == 1 and b"workspace" in L.nsosx_last_error()
