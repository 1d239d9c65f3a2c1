"""The C-ABI library: it loads, exports every symbol include/nsosx.h declares,
and its host-side weight packer matches the oracle (CPU only, no device work)."""
import ctypes

import numpy as np

import reimagined_amd
from reimagined_amd import ops


def test_library_exports_every_header_symbol():
    lib = reimagined_amd.lib()
    names = reimagined_amd.header_symbols()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.nsosx_version().decode().startswith("nsosx")


def test_pack_ternary_matches_oracle(orc):
    rng = np.random.default_rng(11)
    for (n, k) in [(3, 16), (17, 48), (64, 768)]:
        w = rng.standard_normal((n, k)).astype(np.float32)
        packed, ws = ops.pack_ternary(w)
        want_packed, want_ws, codes = orc.pack_weights(w)
        assert ws == want_ws
        np.testing.assert_array_equal(packed, want_packed)
        np.testing.assert_array_equal(ops.unpack_ternary(packed, n * k), codes.ravel())


def test_unpack_reserved_code_decodes_to_zero():
    packed = np.array([0xFFFFFFFF, 0x66666666], np.uint32)
    codes = ops.unpack_ternary(packed, 32)
    assert codes[:16].tolist() == [0] * 16
    assert codes[16:].tolist() == [+1, 0] * 8


def test_pack_rejects_bad_shapes():
    import pytest
    with pytest.raises(ValueError):
        ops.pack_ternary(np.ones((4, 10), np.float32))
    lib = reimagined_amd.lib()
    rc = lib.nsosx_pack_ternary(None, 1, 16, None, None)
    assert rc == 1 and b"null" in lib.nsosx_last_error()


def test_route_workspace_size():
    lib = reimagined_amd.lib()
    assert lib.nsosx_moe_route_workspace(8192, 8) == 32 * 8
    assert lib.nsosx_moe_route_workspace(0, 8) == 0


def _header_param_counts():
    import re
    from reimagined_amd._lib import HEADER
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(nsosx_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_signatures_match_header_arity():
    """The host mirror's hand-kept ctypes table has one entry per header function,
    with the header's parameter count."""
    from reimagined_amd._lib import SIGNATURES
    counts = _header_param_counts()
    assert set(SIGNATURES) == set(counts), set(SIGNATURES) ^ set(counts)
    bad = {n: (len(SIGNATURES[n][1]), c) for n, c in counts.items() if len(SIGNATURES[n][1]) != c}
    assert not bad, bad
