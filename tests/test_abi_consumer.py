"""A compiled C++ consumer of the C ABI (tests/abi_consumer.cpp through the host mirror
reimagined_amd/host/nsosx.hpp).

CPU: the test itself compiles the consumer with g++ -Wall -Wextra -Werror against
include/nsosx.h and the C++ mirror, links it to libnsosx.so, and runs its host-only
mode: the packer against the oracle, the unpacker, SHA-256 against hashlib, the edge
pack parser on a pack written in the reference's layout, and the mapping of a rejected
shape to std::invalid_argument.

GPU: the consumer built by the package build runs BitLinear forward through the C++
mirror on the device: the packed path bit-exact against the oracle, the float
(quantization-sensitive) path within the fp32 bound, and import_packed_state rejecting
a reserved code."""
import hashlib
import json
import os
import subprocess

import numpy as np
import pytest

from edgepack_writer import layer_bytes, pack
from reimagined_amd import build

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _edge_pack(orc, path):
    rng = np.random.default_rng(3)
    w = rng.standard_normal((16, 48)).astype(np.float32)
    packed, ws, _ = orc.pack_weights(w)
    blob = pack([layer_bytes(packed.view(np.uint32), ws, 48, 16,
                             np.ones(16, np.float32), np.zeros(16, np.float32))])
    with open(path, "wb") as fh:
        fh.write(blob)
    return blob, packed


def test_consumer_compiles_warning_free_and_runs_host_entries(tmp_path, orc):
    exe = str(tmp_path / "abi_consumer")
    proc = subprocess.run(build.consumer_cmd(exe), capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    pack_path = str(tmp_path / "layer.pack")
    blob, _ = _edge_pack(orc, pack_path)
    out = subprocess.run([exe, "cpu", pack_path], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, out.stderr
    r = json.loads(out.stdout)
    assert r["version"].startswith("nsosx")
    # the consumer's matrix: LCG ternary codes times a per-element factor (as in the C++)
    N, K = 24, 48
    rr = 20260919
    w = np.empty(N * K, np.float32)
    for i in range(N * K):
        rr = (rr * 1664525 + 1013904223) & 0xFFFFFFFF
        w[i] = np.float32((rr >> 16) % 3 - 1) * np.float32(0.5 + 0.01 * (i % 7))
    want_packed, want_ws, codes = orc.pack_weights(w.reshape(N, K))
    assert r["packed"] == [int(v) for v in want_packed.view(np.uint32)]
    assert r["weight_scale_bits"] == int(np.float32(want_ws).view(np.uint32))
    assert r["code_sum"] == int(codes.astype(np.int64).sum())
    assert r["sha256_abc"] == hashlib.sha256(b"abc").hexdigest()
    assert r["sha256_pack"] == hashlib.sha256(blob).hexdigest()
    assert r["edge_version"] == 3
    assert [(L["in"], L["out"], L["use_bias"], L["sensitive"], L["packed_words"])
            for L in r["edge_layers"]] == [(48, 16, 1, 0, 48)]
    assert r["bad_shape_throws"] == "invalid_argument"


@pytest.mark.gpu
def test_consumer_bitlinear_forward_on_device(dev, orc, tmp_path):
    assert os.path.exists(build.CONSUMER_OUT), "the package build makes the C++ consumer"
    out_path = str(tmp_path / "out.bin")
    proc = subprocess.run([build.CONSUMER_OUT, "gpu", out_path], capture_output=True, text=True,
                          timeout=120)
    assert proc.returncode == 0, proc.stderr
    info = json.loads(proc.stdout)
    M, K, N = info["M"], info["K"], info["N"]
    data = np.fromfile(out_path, np.float32)
    sizes = [M * K, N * K, N, N, M * N, M * N]
    parts = np.split(data, np.cumsum(sizes)[:-1])
    x, w, mag, bias, y_packed, y_float = (p.copy() for p in parts)
    x, w = x.reshape(M, K), w.reshape(N, K)
    packed, ws, _ = orc.pack_weights(w)
    want = orc.bitlinear_forward(x, packed, ws, N, 8, True, mag, bias)
    np.testing.assert_array_equal(y_packed.reshape(M, N).view(np.uint32), want.view(np.uint32))
    want_f = orc.linear_f32(x, w, True, mag, bias)
    np.testing.assert_allclose(y_float.reshape(M, N), want_f, rtol=1e-4,
                               atol=1e-5 * np.abs(want_f).max())
    assert info["reserved_code_import"] == "invalid_argument"
