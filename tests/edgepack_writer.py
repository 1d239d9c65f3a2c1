"""Test helper: writes edge linear packs in the reference's layout
(JambaModel::save_edge_linear_pack, OXN/nsos/src/jamba.cpp:1325-1445; write_pod /
write_vector 504-536): u32 magic, u32 version, u32 count, per layer u8 sensitive,
i32 in, i32 out, u8 use_bias, f32 weight_scale, then u64-counted vectors
packed_weights, magnitude, bias, flat_alpha, flat_beta (+ fp32 weights when
sensitive); version 3 appends u32 "EGI3", u64 payload bytes, 64 hex SHA-256."""
import hashlib
import struct

import numpy as np

MAGIC = 0x31454744
TRAILER = 0x33494745


def _vec(arr, dtype):
    a = np.ascontiguousarray(arr, dtype=dtype)
    return struct.pack("<Q", a.size) + a.tobytes()


def layer_bytes(packed_u32, ws, n_in, n_out, magnitude, bias=None, alpha=None, beta=None,
                sensitive_w=None):
    alpha = np.ones(n_in, np.float32) if alpha is None else alpha
    beta = np.zeros(n_in, np.float32) if beta is None else beta
    out = struct.pack("<BiiBf", 1 if sensitive_w is not None else 0, n_in, n_out,
                      1 if bias is not None else 0, ws)
    out += _vec(packed_u32, np.uint32) + _vec(magnitude, np.float32)
    out += _vec(np.zeros(0, np.float32) if bias is None else bias, np.float32)
    out += _vec(alpha, np.float32) + _vec(beta, np.float32)
    if sensitive_w is not None:
        out += _vec(np.asarray(sensitive_w).ravel(), np.float32)
    return out


def pack(layers, version=3):
    payload = struct.pack("<III", MAGIC, version, len(layers)) + b"".join(layers)
    if version < 3:
        return payload
    digest = hashlib.sha256(payload).hexdigest().encode()
    return payload + struct.pack("<IQ", TRAILER, len(payload)) + digest
