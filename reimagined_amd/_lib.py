"""ctypes binding of libnsosx.so (the C ABI declared in include/nsosx.h).

The library is loaded from this package directory only; a missing library is
an error, never a fallback.  Symbol signatures mirror the header one to one.
"""
from __future__ import annotations

import ctypes
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libnsosx.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "nsosx.h")

_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

SIGNATURES = {
    "nsosx_last_error": (ctypes.c_char_p, []),
    "nsosx_version": (ctypes.c_char_p, []),
    "nsosx_pack_ternary": (_i, [_vp, _i, _i, _vp, _vp]),
    "nsosx_unpack_ternary": (_i, [_vp, _i64, _vp]),
    "nsosx_find_reserved_code": (_i, [_vp, _i64, _vp, _vp]),
    "nsosx_weight_row_sums": (_i, [_vp, _i, _i, _vp, _vp]),
    "nsosx_quantize_act_i8": (_i, [_vp, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "nsosx_ternary_gemm": (_i, [_vp, _vp, _vp, _f, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "nsosx_ternary_gemm_path": (_i, [_vp, _vp, _vp, _f, _i, _i, _i, _vp, _vp, _vp, _i, _vp,
                                     _i, _vp]),
    "nsosx_bitlinear_forward": (_i, [_vp, _i, _vp, _f, _i, _i, _i, _i, _i, _vp, _vp, _vp, _i,
                                     _vp, _vp, _vp, _vp]),
    "nsosx_bitlinear_forward_noalloc_max_bytes": (_i64, []),
    "nsosx_bitlinear_forward_noalloc": (_i, [_vp, _i, _vp, _f, _i, _i, _i, _i, _i, _vp, _vp,
                                             _vp, _i, _vp]),
    "nsosx_linear_f32": (_i, [_vp, _i, _i, _i, _vp, _i, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "nsosx_bitlinear_ste_backward_workspace": (_i64, [_i, _i, _i, _i]),
    "nsosx_bitlinear_ste_backward": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _f, _i, _i, _i, _i, _vp,
                                          _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "nsosx_pack_mfma_layout": (_i, [_vp, _i64, _vp, _vp]),
    "nsosx_ternary_gemm_mfma": (_i, [_vp, _vp, _vp, _f, _i, _i, _i, _vp, _vp, _vp, _i, _vp, _vp]),
    "nsosx_grouped_ternary_gemm_mfma": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i,
                                             _vp, _i, _vp]),
    "nsosx_grouped_ternary_gemm_mfma_workspace": (_i64, []),
    "nsosx_grouped_ternary_gemm_mfma_ws": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i,
                                                _vp, _i, _vp, _i64, _vp]),
    "nsosx_grouped_gemv": (_i, [_vp, _i, _vp, _i64, _vp, _i64, _i, _vp, _i64, _i, _vp]),
    "nsosx_grouped_decode_projections": (_i, [_vp, _i, _vp, _i, _vp, _i64, _i, _vp]),
    "nsosx_conv1d_causal": (_i, [_vp, _i, _i64, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp, _i,
                                 _vp]),
    "nsosx_selective_scan_fwd": (_i, [_vp, _i64, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i64, _vp,
                                      _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "nsosx_conv_scan_fwd": (_i, [_vp, _i64, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i64,
                                 _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "nsosx_scan_fwd_workspace": (_i64, [_i, _i, _i, _i, _i, _i]),
    "nsosx_scan_fwd_planned": (_i, [_vp, _i64, _vp, _vp, _i, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                                    _i64, _vp, _i, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _i,
                                    _vp, _vp]),
    "nsosx_selective_scan_step": (_i, [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                       _i, _i, _vp, _vp, _vp]),
    "nsosx_mamba2_step": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i, _vp, _vp, _vp, _vp,
                               _f, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp]),
    "nsosx_mamba2_step_out": (_i, [_vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i, _vp, _vp, _vp,
                                   _vp, _f, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _i, _vp,
                                   _f, _i, _vp, _vp, _vp, _i, _vp]),
    "nsosx_moe_route_workspace": (_i64, [_i, _i]),
    "nsosx_moe_route": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                             _vp]),
    "nsosx_grouped_ternary_gemm": (_i, [_vp, _i, _vp, _vp, _i, _vp, _vp, _i, _i, _i, _i, _i,
                                        _vp, _i, _vp]),
    "nsosx_moe_combine": (_i, [_vp, _i, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _i, _vp]),
    "nsosx_rmsnorm_gated": (_i, [_vp, _vp, _vp, _i, _i, _f, _i, _vp, _i, _vp]),
    "nsosx_rmsnorm_gated_quant": (_i, [_vp, _vp, _vp, _i, _i, _f, _i, _vp, _i, _i, _vp, _vp,
                                       _vp]),
    "nsosx_add_rmsnorm": (_i, [_vp, _vp, _vp, _i, _i, _f, _i, _vp, _vp, _vp]),
    "nsosx_conv_step": (_i, [_vp, _i, _i64, _i, _i, _vp, _vp, _i, _vp, _i, _vp, _i, _vp]),
    "nsosx_edge_pack_parse": (_i, [_vp, ctypes.c_uint64, _vp, _i, _vp, _vp]),
    "nsosx_qat_fake_quant_ternary": (_i, [_vp, _i64, ctypes.c_float, _vp, _vp]),
    "nsosx_qat_absmean_workspace": (_i64, [_i64]),
    "nsosx_qat_fake_quant_ternary_absmean": (_i, [_vp, _i64, _vp, _vp, _vp, _vp]),
    "nsosx_qat_fake_quant_activations": (_i, [_vp, _i, _i, _i, _vp, _vp]),
    "nsosx_qat_ste_clip_weight_grad": (_i, [_vp, _vp, _i64, ctypes.c_float, _vp, _vp]),
    "nsosx_moe_sparse_decode_workspace": (_i64, [_i, _i, _i, _i]),
    "nsosx_moe_sparse_decode": (_i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp,
                                     _vp, _i, _vp]),
    "nsosx_sha256_hex": (_i, [_vp, ctypes.c_uint64, _vp]),
}

STATUS = {0: "OK", 1: "INVALID", 2: "OVERFLOW", 3: "RESERVED", 4: "LAUNCH"}


class NsosxError(RuntimeError):
    def __init__(self, fn: str, status: int, text: str):
        super().__init__(f"{fn} failed ({STATUS.get(status, status)}): {text}")
        self.status = status


_lib = None


def header_symbols() -> list[str]:
    """Every function the C header declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(nsosx_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m reimagined_amd.build` "
                "(there is no fallback path)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def call(name: str, *args) -> None:
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        text = lib().nsosx_last_error().decode()
        if rc == 1:
            raise ValueError(f"{name}: {text}")
        raise NsosxError(name, rc, text)
