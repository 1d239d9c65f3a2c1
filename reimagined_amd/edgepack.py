"""Edge linear pack loader: the reference's on-disk BitLinear format ("DGE1" v3 with
its "EGI3" SHA-256 trailer, or legacy v2) straight into device-resident layers.

JambaModel::load_edge_linear_pack (OXN/nsos/src/jamba.cpp:1447-1620) parses, validates
and stages every layer before committing; here the C ABI (nsosx_edge_pack_parse) does
the parse and validation on the host buffer, and each packed layer's words go to the
device unchanged (they are the format the GEMM/GEMV kernels read).  Layers the pack
marks quantization-sensitive carry fp32 weights for the reference's float path, which
this build does not run: they are returned as EdgeFloatLayer records, not BitLinears.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from ._lib import call, lib


class EdgeLayer(ctypes.Structure):
    _fields_ = [("in_features", ctypes.c_int32), ("out_features", ctypes.c_int32),
                ("use_bias", ctypes.c_int32), ("sensitive", ctypes.c_int32),
                ("weight_scale", ctypes.c_float), ("packed_words", ctypes.c_uint64),
                ("packed_offset", ctypes.c_uint64), ("magnitude_offset", ctypes.c_uint64),
                ("bias_offset", ctypes.c_uint64), ("alpha_offset", ctypes.c_uint64),
                ("beta_offset", ctypes.c_uint64), ("sensitive_offset", ctypes.c_uint64)]


@dataclass
class EdgeFloatLayer:
    """A quantization-sensitive layer: fp32 weight [out, in] (+ bias) for the float path."""
    weight: np.ndarray
    bias: np.ndarray | None


def parse(buf) -> tuple[int, list]:
    """Validates a pack held in memory -> (version, [EdgeLayer]) (offsets into buf)."""
    data = np.frombuffer(buf, dtype=np.uint8)
    ptr = data.ctypes.data_as(ctypes.c_void_p)
    n = ctypes.c_int(0)
    ver = ctypes.c_uint32(0)
    rc = lib().nsosx_edge_pack_parse(ptr, data.size, None, 0, ctypes.byref(n), ctypes.byref(ver))
    if rc not in (0, 2):  # 2: more layers than descriptors (the count query)
        call("nsosx_edge_pack_parse", ptr, data.size, None, 0, ctypes.byref(n), ctypes.byref(ver))
    layers = (EdgeLayer * max(n.value, 1))()
    call("nsosx_edge_pack_parse", ptr, data.size, layers, n.value, ctypes.byref(n),
         ctypes.byref(ver))
    return ver.value, [layers[i] for i in range(n.value)]


def sha256_hex(buf) -> str:
    data = np.frombuffer(buf, dtype=np.uint8)
    out = ctypes.create_string_buffer(65)
    call("nsosx_sha256_hex", data.ctypes.data_as(ctypes.c_void_p), data.size, out)
    return out.value.decode()


def load(path: str, device="cuda", bits: int = 8, rms_input: bool = True) -> list:
    """Reads a pack file -> one entry per layer, in file order: a device BitLinear for
    packed layers, an EdgeFloatLayer for sensitive ones."""
    from .layers import BitLinear
    buf = np.fromfile(path, dtype=np.uint8)
    _, descs = parse(buf)
    out = []
    for d in descs:
        f32 = lambda off, cnt: buf[off:off + 4 * cnt].view(np.float32).copy()
        bias = f32(d.bias_offset, d.out_features) if d.use_bias else None
        if d.sensitive:
            w = f32(d.sensitive_offset, d.out_features * d.in_features)
            out.append(EdgeFloatLayer(w.reshape(d.out_features, d.in_features), bias))
            continue
        if d.in_features % 16:
            raise ValueError("edge pack layer: the device GEMM needs in_features % 16 == 0")
        words = buf[d.packed_offset:d.packed_offset + 4 * d.packed_words].view(np.uint32)
        mag = torch.from_numpy(f32(d.magnitude_offset, d.out_features)).to(device)
        layer = BitLinear.from_packed(words, d.weight_scale, d.out_features, d.in_features,
                                      device, bits=bits, rms_input=rms_input, magnitude=mag,
                                      bias=None if bias is None else torch.from_numpy(bias).to(device))
        layer.flat_alpha = f32(d.alpha_offset, d.in_features)
        layer.flat_beta = f32(d.beta_offset, d.in_features)
        out.append(layer)
    return out
