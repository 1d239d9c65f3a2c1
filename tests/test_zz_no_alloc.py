"""The allocation-free BitLinear forward (library-owned scratch) against the
caller-workspace entry point it shares its kernels with: bit-exact outputs on
two calls in a row, the second with a smaller input (the scratch keeps the
first call's contents), the same under HIP graph capture and replay, and the
size limit rejected with a clear error."""
import numpy as np
import pytest
import torch

from reimagined_amd import ops
from reimagined_amd._lib import lib

pytestmark = pytest.mark.gpu


def _noalloc():
    return lib().nsosx_bitlinear_forward_noalloc


def _run_noalloc(x, packed, ws, n, rms, mag, bias, out_dtype):
    m, k = x.shape
    y = torch.empty((m, n), dtype=out_dtype, device=x.device)
    rc = _noalloc()(ops._p(x), ops._dt(x), ops._p(packed), ws, m, k, n, 8, int(rms), ops._p(mag),
                    ops._p(bias), ops._p(y), ops._DT[out_dtype], ops._stream())
    assert rc == 0, lib().nsosx_last_error().decode()
    return y


@pytest.mark.parametrize("rms,xdt,ydt", [(True, torch.float32, torch.float32),
                                         (False, torch.bfloat16, torch.bfloat16)])
def test_noalloc_matches_workspace_entry(dev, rms, xdt, ydt):
    rng = np.random.default_rng(11)
    k, n = 1024, 640
    w = rng.standard_normal((n, k)).astype(np.float32)
    packed, ws = ops.pack_ternary(w)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    mag = torch.from_numpy(rng.uniform(0.5, 1.5, n).astype(np.float32)).to(dev)
    bias = torch.from_numpy(rng.standard_normal(n).astype(np.float32)).to(dev)
    for m in (300, 5):   # the second call is smaller: stale scratch from the first must not leak
        x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev).to(xdt)
        got = _run_noalloc(x, pk, ws, n, rms, mag, bias, ydt)
        want = ops.bitnet_gemm_158bit_gpu(x, pk, ws, m, k, n, 8, mag, bias, rms_input=rms,
                                          out_dtype=ydt)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"m={m}"


def test_noalloc_rejects_oversize(dev):
    limit = int(lib().nsosx_bitlinear_forward_noalloc_max_bytes())
    k = 4096
    m = limit // k + 1
    packed = torch.zeros(16 * k // 16, dtype=torch.int32, device=dev)
    x = torch.zeros((1, k), dtype=torch.float32, device=dev)
    y = torch.zeros((1, 16), dtype=torch.float32, device=dev)
    # the size check runs before anything is enqueued; no pointer is dereferenced
    rc = _noalloc()(ops._p(x), 0, ops._p(packed), 1.0, m, k, 16, 8, 0, None, None, ops._p(y), 0,
                    ops._stream())
    assert rc == 2
    assert "scratch" in lib().nsosx_last_error().decode()


def test_noalloc_captured_in_graph(dev):
    """The documented use: a noalloc call captured into a HIP graph (after one eager call on
    the device, which looks the scratch address up) and replayed; every replay, with eager
    work of other shapes on the same scratch in between, is bit-exact with the
    caller-workspace entry."""
    rng = np.random.default_rng(12)
    k, n, m = 2048, 512, 64
    w = rng.standard_normal((n, k)).astype(np.float32)
    packed, ws = ops.pack_ternary(w)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    x = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float32)).to(dev)
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    fwd = _noalloc()

    def run():
        return fwd(ops._p(x), ops._dt(x), ops._p(pk), ws, m, k, n, 8, 1, None, None, ops._p(y),
                   ops._DT[torch.float32], ops._stream())
    assert run() == 0, lib().nsosx_last_error().decode()  # eager first call on the device
    torch.cuda.synchronize()
    want = ops.bitnet_gemm_158bit_gpu(x, pk, ws, m, k, n, 8, None, None, rms_input=True,
                                      out_dtype=torch.float32)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rc = run()
    torch.cuda.current_stream().wait_stream(s)
    assert rc == 0, lib().nsosx_last_error().decode()
    other = torch.from_numpy(rng.standard_normal((300, k)).astype(np.float32)).to(dev)
    for rep in range(4):
        y.fill_(float("nan"))
        # eager noalloc work of another shape leaves other contents in the scratch
        _run_noalloc(other, pk, ws, n, True, None, None, torch.float32)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want), f"replay {rep}"
