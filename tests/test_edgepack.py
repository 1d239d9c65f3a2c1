"""Edge linear pack parsing through the C ABI on the host (no GPU): the SHA-256 the
trailer carries against hashlib, a round trip of packs written in the reference's
layout (tests/edgepack_writer.py), and every rejection of load_edge_linear_pack
(OXN/nsos/src/jamba.cpp:1447-1620, 556-616)."""
import hashlib
import struct

import numpy as np
import pytest

from reimagined_amd import edgepack
from reimagined_amd._lib import NsosxError
from edgepack_writer import layer_bytes, pack


@pytest.mark.parametrize("n", [0, 1, 3, 55, 56, 57, 63, 64, 65, 119, 120, 1000, 1 << 20])
def test_sha256_matches_hashlib(n):
    data = np.random.default_rng(n).integers(0, 256, n, dtype=np.uint8).tobytes()
    assert edgepack.sha256_hex(data) == hashlib.sha256(data).hexdigest()


def _layers(orc, rng):
    out = []
    specs = [(64, 32, False, False), (48, 16, True, False), (32, 8, True, True)]
    for n_in, n_out, use_bias, sensitive in specs:
        w = rng.standard_normal((n_out, n_in)).astype(np.float32)
        packed, ws, _ = orc.pack_weights(w)
        mag = rng.uniform(0.5, 1.5, n_out).astype(np.float32)
        bias = rng.standard_normal(n_out).astype(np.float32) if use_bias else None
        alpha = rng.standard_normal(n_in).astype(np.float32)
        beta = rng.standard_normal(n_in).astype(np.float32)
        out.append(dict(packed=packed.view(np.uint32), ws=ws, n_in=n_in, n_out=n_out, mag=mag,
                        bias=bias, alpha=alpha, beta=beta, w=w if sensitive else None))
    return out


def _bytes(ls):
    return [layer_bytes(l["packed"], l["ws"], l["n_in"], l["n_out"], l["mag"], l["bias"],
                        l["alpha"], l["beta"], l["w"]) for l in ls]


@pytest.mark.parametrize("version", [2, 3])
def test_round_trip(orc, version):
    ls = _layers(orc, np.random.default_rng(1))
    buf = pack(_bytes(ls), version)
    ver, descs = edgepack.parse(buf)
    assert ver == version and len(descs) == len(ls)
    b = np.frombuffer(buf, np.uint8)
    for d, l in zip(descs, ls):
        assert (d.in_features, d.out_features) == (l["n_in"], l["n_out"])
        assert d.weight_scale == l["ws"] and d.use_bias == (l["bias"] is not None)
        assert d.sensitive == (l["w"] is not None)
        words = b[d.packed_offset:d.packed_offset + 4 * d.packed_words].view(np.uint32)
        np.testing.assert_array_equal(words, l["packed"])
        f = lambda off, n: b[off:off + 4 * n].view(np.float32)
        np.testing.assert_array_equal(f(d.magnitude_offset, d.out_features), l["mag"])
        np.testing.assert_array_equal(f(d.alpha_offset, d.in_features), l["alpha"])
        np.testing.assert_array_equal(f(d.beta_offset, d.in_features), l["beta"])
        if l["bias"] is not None:
            np.testing.assert_array_equal(f(d.bias_offset, d.out_features), l["bias"])
        if l["w"] is not None:
            np.testing.assert_array_equal(f(d.sensitive_offset, d.in_features * d.out_features),
                                          l["w"].ravel())


def _corrupt(buf, pos, value_bytes, refresh_trailer=True):
    b = bytearray(buf)
    b[pos:pos + len(value_bytes)] = value_bytes
    if refresh_trailer:  # keep the trailer valid so the field check itself is reached
        payload = bytes(b[:-76])
        b[-64:] = hashlib.sha256(payload).hexdigest().encode()
    return bytes(b)


def test_rejections(orc):
    ls = _layers(orc, np.random.default_rng(2))
    good = pack(_bytes(ls), 3)
    cases = {
        "magic": _corrupt(good, 0, b"XXXX"),
        "version": _corrupt(good, 4, struct.pack("<I", 4)),
        "sha": _corrupt(good, 40, b"\x01", refresh_trailer=False),
        "trailer_len": _corrupt(good, len(good) - 72, struct.pack("<Q", 5), refresh_trailer=False),
        "truncated": good[:-1],
        "sensitivity_flag": _corrupt(good, 12, b"\x02"),
        "weight_scale": _corrupt(good, 22, struct.pack("<f", 0.0)),
        "count": _corrupt(good, 26, struct.pack("<Q", 7)),
        "trailing_v2": pack(_bytes(ls), 2) + b"\x00",
    }
    for name, buf in cases.items():
        with pytest.raises(ValueError):
            edgepack.parse(buf)
    # a non-finite magnitude
    l0 = dict(ls[0])
    l0["mag"] = l0["mag"].copy()
    l0["mag"][3] = np.inf
    with pytest.raises(ValueError):
        edgepack.parse(pack(_bytes([l0]), 3))
    # the reserved code 3 is its own status
    l1 = dict(ls[0])
    l1["packed"] = l1["packed"].copy()
    l1["packed"][5] |= 0x3 << 8
    with pytest.raises(NsosxError) as e:
        edgepack.parse(pack(_bytes([l1]), 3))
    assert e.value.status == 3
