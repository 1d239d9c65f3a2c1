"""Host-side argument checks of the scan wrappers (CPU only).

The C ABI receives raw device pointers, so every tensor's shape has to be
checked on the host before a call: an undersized state, dt, B, C, D, a_log or
conv weight would otherwise be read or written out of bounds on the device.
These run on CPU tensors; a wrapper must reject the bad shape with ValueError
before it looks at the device, and a well-shaped CPU tensor gets as far as
the device check."""
import numpy as np
import pytest
import torch

from reimagined_amd import ops

T, H, P, N, G = 10, 4, 2, 16, 2


def _good():
    f = torch.float32
    return dict(x=torch.zeros(T, H * P, dtype=f), dt=torch.zeros(T, H, dtype=f),
                a_log=torch.zeros(H, N, dtype=f), B=torch.zeros(T, G * N, dtype=f),
                C=torch.zeros(T, G * N, dtype=f), D=torch.zeros(H, dtype=f),
                z=torch.zeros(T, H * P, dtype=f), cu=torch.tensor([0, 4, T], dtype=torch.int32),
                conv_w=torch.zeros(H * P, 4, dtype=f), conv_b=torch.zeros(H * P, dtype=f),
                state=torch.zeros(3, H * P, N, dtype=f), init=torch.zeros(2, H * P, N, dtype=f))


def _fwd(a):
    return ops.selective_scan_fwd(a["x"], a["dt"], a["a_log"], a["B"], a["C"], a["D"], a["z"],
                                  a["cu"], H, P, N, G, initial_state=a["init"])


def _conv_scan(a):
    return ops.conv_scan_fwd(a["x"], a["conv_w"], a["conv_b"], a["dt"], a["a_log"], a["B"],
                             a["C"], a["D"], a["z"], a["cu"], H, P, N, G,
                             initial_state=a["init"])


def _step(a):
    r = a["state"].shape[0]
    return ops.selective_scan_step(a["x"][:r], a["dt"][:r], a["a_log"], a["B"][:r], a["C"][:r],
                                   a["D"], a["z"][:r], a["state"], H, P, N, G)


BAD = [
    ("x", torch.zeros(T, H * P + 1)),
    ("dt", torch.zeros(T - 1, H)),
    ("dt", torch.zeros(T, H - 1)),
    ("B", torch.zeros(T, G * N - 1)),
    ("C", torch.zeros(T - 1, G * N)),
    ("z", torch.zeros(T, H * P - 2)),
    ("D", torch.zeros(H - 1)),
    ("a_log", torch.zeros(H, N - 1)),
    ("init", torch.zeros(1, H * P, N)),
    ("init", torch.zeros(2, H * P, N - 1)),
]


@pytest.mark.parametrize("name,bad", BAD)
@pytest.mark.parametrize("fn", [_fwd, _conv_scan])
def test_prefill_rejects_bad_shapes(fn, name, bad):
    a = _good()
    a[name] = bad
    with pytest.raises(ValueError, match=name if name != "init" else "initial_state"):
        fn(a)


@pytest.mark.parametrize("name,bad", [("conv_w", torch.zeros(H * P - 1, 4)),
                                      ("conv_w", torch.zeros(H * P, 9)),
                                      ("conv_b", torch.zeros(H * P + 1)),
                                      ("cu", torch.zeros(1, dtype=torch.int32))])
def test_conv_scan_rejects_bad_conv_and_offsets(name, bad):
    a = _good()
    a[name] = bad
    with pytest.raises(ValueError):
        _conv_scan(a)


@pytest.mark.parametrize("name,bad", [("state", torch.zeros(3, H * P, N - 1)),
                                      ("state", torch.zeros(3, H * P - 1, N)),
                                      ("D", torch.zeros(H + 1))])
def test_step_rejects_bad_shapes(name, bad):
    a = _good()
    a[name] = bad
    with pytest.raises(ValueError, match=name):
        _step(a)


@pytest.mark.parametrize("fn", [_fwd, _conv_scan, _step])
def test_well_shaped_cpu_tensors_reach_the_device_check(fn):
    with pytest.raises(ValueError, match="device tensor"):
        fn(_good())


def test_mfma_layout_gemm_rejects_k_past_int32_range():
    """MFMA-layout operands carry 64 x the ternary values, so the int32 sums hold
    64 * 127 * K at most: K past 2^31 / (64 * 127) is refused before any device work
    (the pointers here are host placeholders and are never dereferenced)."""
    import ctypes
    import numpy as np
    from reimagined_amd import _lib
    lib = _lib.lib()
    buf = np.zeros(64, np.uint8)
    base = buf.ctypes.data
    p = ctypes.c_void_p((base + 15) & ~15)  # 16-byte aligned placeholder
    k_big = ((2147483647 // (64 * 127)) // 128 + 1) * 128
    f = lib.nsosx_ternary_gemm_mfma
    f.restype = ctypes.c_int
    rc = f(p, p, p, ctypes.c_float(1.0), 1, k_big, 16, None, None, p, 1, None, None)
    assert rc == 2, lib.nsosx_last_error().decode()   # NSOSX_ERR_OVERFLOW
    assert "64x-scaled" in lib.nsosx_last_error().decode()


# ---- C-ABI argument checks that run before anything touches the device --------------
# The pointers below are non-null placeholders: each call is refused by its argument
# checks, which run before any pointer is dereferenced or any launch is made.
_FAKE = 1 << 20  # a 256-byte-aligned placeholder address, never dereferenced


def test_planned_scan_rejects_bad_group_count():
    """G == 0 (or H % G != 0) is NSOSX_ERR_INVALID, not a host divide-by-zero."""
    from reimagined_amd._lib import lib
    L = lib()
    for G in (0, 3):
        rc = L.nsosx_scan_fwd_planned(_FAKE, 0, None, None, 0, _FAKE, _FAKE, 1, _FAKE, _FAKE,
                                      _FAKE, None, 0, _FAKE, 2, 100, 4, 16, 16, G, 0, None, None,
                                      _FAKE, -1, _FAKE, None)
        assert rc == 1, (G, rc)
        assert b"H % G" in L.nsosx_last_error()


def test_grouped_mfma_gemm_requires_total_rows():
    """total_rows == 0 is refused (the MFMA-layout grouped GEMM sizes its grid from it),
    where it used to return success with the output untouched."""
    from reimagined_amd._lib import lib
    L = lib()
    rc = L.nsosx_grouped_ternary_gemm_mfma(_FAKE, 8, _FAKE, _FAKE, 1, _FAKE, _FAKE, 1024, 4096,
                                           0, 1, _FAKE, 1, None)
    assert rc == 1
    assert b"total_rows > 0" in L.nsosx_last_error()


def test_moe_route_argument_checks():
    from reimagined_amd._lib import lib
    L = lib()
    # k above E, E above 64, and partial null outputs
    rc = L.nsosx_moe_route(_FAKE, None, 16, 16, 17, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE,
                           None, _FAKE, None)
    assert rc == 1 and b"k <= E" in L.nsosx_last_error()
    rc = L.nsosx_moe_route(_FAKE, None, 16, 65, 2, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE, _FAKE,
                           None, _FAKE, None)
    assert rc == 1
    rc = L.nsosx_moe_route(_FAKE, None, 16, 8, 2, _FAKE, _FAKE, _FAKE, None, None, None, None,
                           None, None)
    assert rc == 1 and b"null pointer" in L.nsosx_last_error()


def test_moe_route_host_mask_validation():
    """The host mirror checks a host mask as MoERouter::forward does (src/jamba.cpp:
    8145-8153) before touching the device."""
    from reimagined_amd.ops import valid_rows_mask
    with pytest.raises(ValueError, match="only 0 or 1"):
        valid_rows_mask([1, 0, 2], 3, "cpu")
    with pytest.raises(ValueError, match="size mismatch"):
        valid_rows_mask([1, 0], 3, "cpu")
    assert valid_rows_mask(None, 3, "cpu") is None
    assert valid_rows_mask([], 3, "cpu") is None
    m = valid_rows_mask(np.array([1, 0, 1]), 3, "cpu")
    assert m.dtype == torch.uint8 and m.tolist() == [1, 0, 1]


def test_grouped_mfma_ws_argument_checks():
    """The split-K tail entry checks its workspace pointer and the shapes before it asks the
    device anything (no device here)."""
    from reimagined_amd._lib import lib
    L = lib()
    rc = L.nsosx_grouped_ternary_gemm_mfma_ws(_FAKE, 8, _FAKE, _FAKE, 1, _FAKE, _FAKE, 1024,
                                              4096, 100, 1, _FAKE, 1, None, 1 << 26, None)
    assert rc == 1 and b"null pointer" in L.nsosx_last_error()
    rc = L.nsosx_grouped_ternary_gemm_mfma_ws(_FAKE, 8, _FAKE, _FAKE, 1, _FAKE, _FAKE, 1024,
                                              4096, 0, 1, _FAKE, 1, _FAKE, 1 << 26, None)
    assert rc == 1 and b"total_rows > 0" in L.nsosx_last_error()
    rc = L.nsosx_grouped_ternary_gemm_mfma_ws(_FAKE, 8, _FAKE, _FAKE, 1, _FAKE, _FAKE, 1000,
                                              4096, 100, 1, _FAKE, 1, _FAKE, 1 << 26, None)
    assert rc == 1 and b"K % 128" in L.nsosx_last_error()
