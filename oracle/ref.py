"""numpy front end of oracle/_ref/libnsos_ref.so: the reference's own compiled operators.

TEST INFRASTRUCTURE ONLY: the library is built from the reference's sources by
`make -C oracle ref` where the reference tree is mounted.  tests/golden/
gen_golden.py records its outputs as fixtures (the tests compare the oracle,
and through it the GPU path, against those fixtures, so no test needs the
reference itself), and bench.py's cpu_baseline leg times its BitLinear forward
as the reference's CPU path when the built library is present.

Every wrapper names the reference function it calls (paths under OXN/nsos/).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
REF_PATH = os.path.join(_HERE, "_ref", "libnsos_ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float

_lib = None


def available() -> bool:
    return os.path.exists(REF_PATH)


def _load():
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(REF_PATH)
        sig = {
            "ref_last_error": (ctypes.c_char_p, []),
            "ref_rmsnorm": (_i, [_f32p, _i, _i, _f, _f32p]),
            "ref_softmax": (_i, [_f32p, _i, _i, _f32p]),
            "ref_silu": (_i, [_f32p, _i64, _f32p]),
            "ref_silu_gate": (_i, [_f32p, _f32p, _i64, _f32p]),
            "ref_squared_relu": (_i, [_f32p, _i64, _f32p]),
            "ref_abs_mean": (_i, [_f32p, _i64, ctypes.POINTER(_f)]),
            "ref_rmsnorm_backward": (_i, [_f32p, _f32p, _f32p, _i, _i, _f, _f32p]),
            "ref_bitlinear_forward": (_i, [_f32p, _i, _i, _f32p, _i, _i, _vp, _vp, _i, _f32p]),
            "ref_bitlinear_packed_backward": (_i, [_f32p, _i, _i, _f32p, _i, _i, _vp, _vp,
                                                   _f32p, _f32p, _f32p, _f32p, _vp, _vp]),
            "ref_bitlinear_time_forward": (_i, [_f32p, _i, _i, _f32p, _i, _i, _i, _f32p,
                                                ctypes.POINTER(ctypes.c_double)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: reference threw: {_load().ref_last_error().decode()}")


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def rmsnorm(x, eps: float = 1e-6):
    """Tensor::rmsnorm (src/tensor.cpp:3455-3492)."""
    x = _f32(x)
    out = np.empty_like(x)
    _check(_load().ref_rmsnorm(x, x.shape[0], x.shape[1], eps, out), "rmsnorm")
    return out


def softmax(x):
    """Tensor::softmax(-1) (src/tensor.cpp:3402-3453)."""
    x = _f32(x)
    out = np.empty_like(x)
    _check(_load().ref_softmax(x, x.shape[0], x.shape[1], out), "softmax")
    return out


def silu(x):
    """Tensor::silu (src/tensor.cpp:3261-3282)."""
    x = _f32(x)
    out = np.empty_like(x)
    _check(_load().ref_silu(x.ravel(), x.size, out.ravel()), "silu")
    return out


def silu_gate(v, g):
    """Tensor::silu_gate (src/tensor.cpp:3323-3343): v * silu(g)."""
    v, g = _f32(v), _f32(g)
    out = np.empty_like(v)
    _check(_load().ref_silu_gate(v.ravel(), g.ravel(), v.size, out.ravel()), "silu_gate")
    return out


def squared_relu(x):
    """Tensor::squared_relu (src/tensor.cpp:3209-3226)."""
    x = _f32(x)
    out = np.empty_like(x)
    _check(_load().ref_squared_relu(x.ravel(), x.size, out.ravel()), "squared_relu")
    return out


def abs_mean(w) -> np.float32:
    """tensor_abs_mean (src/tensor.cpp:2072-2107)."""
    w = _f32(w)
    out = ctypes.c_float()
    _check(_load().ref_abs_mean(w.ravel(), w.size, ctypes.byref(out)), "abs_mean")
    return np.float32(out.value)


def rmsnorm_backward(x, grad, x_norm, eps: float = 1e-6):
    """Tensor::rmsnorm_backward (src/tensor.cpp:3997-4056)."""
    x, grad, x_norm = _f32(x), _f32(grad), _f32(x_norm)
    out = np.empty_like(x)
    _check(_load().ref_rmsnorm_backward(x, grad, x_norm, x.shape[0], x.shape[1], eps, out),
           "rmsnorm_backward")
    return out


def bitlinear_forward(w, x, packed: bool = True, exact_linear: bool = False, magnitude=None,
                      bias=None):
    """BitLinear::forward on the CPU (src/bitlinear.cpp:439-741): packed ternary path or
    the float reference path; default RMS_PERI + magnitude, or exact-linear mode."""
    w, x = _f32(w), _f32(x)
    n, k = w.shape
    m = x.shape[0]
    mag = None if magnitude is None else _f32(magnitude)
    b = None if bias is None else _f32(bias)
    y = np.empty((m, n), np.float32)
    _check(_load().ref_bitlinear_forward(w, n, k, x, m, int(exact_linear), _ptr(mag), _ptr(b),
                                         int(packed), y), "bitlinear_forward")
    return y


def bitlinear_packed_backward(w, x, grad, exact_linear: bool = False, magnitude=None,
                              bias=None) -> dict:
    """BitLinear forward + STE backward on the packed path (src/bitlinear.cpp:1191-1357)."""
    w, x, grad = _f32(w), _f32(x), _f32(grad)
    n, k = w.shape
    m = x.shape[0]
    mag = None if magnitude is None else _f32(magnitude)
    b = None if bias is None else _f32(bias)
    out = {"y": np.empty((m, n), np.float32), "dx": np.empty((m, k), np.float32),
           "dW": np.empty((n, k), np.float32)}
    dmag = None if exact_linear else np.empty(n, np.float32)
    dbias = None if bias is None else np.empty(n, np.float32)
    _check(_load().ref_bitlinear_packed_backward(w, n, k, x, m, int(exact_linear), _ptr(mag),
                                                 _ptr(b), grad, out["y"], out["dx"], out["dW"],
                                                 _ptr(dmag), _ptr(dbias)),
           "bitlinear_packed_backward")
    if dmag is not None:
        out["dmag"] = dmag
    if dbias is not None:
        out["dbias"] = dbias
    return out


def bitlinear_time_forward(w, x, exact_linear: bool = False, reps: int = 1):
    """Seconds per BitLinear::forward call on the CPU packed path (one configured layer,
    packing outside the timed loop) and the last output: the reference's own CPU hot path."""
    w, x = _f32(w), _f32(x)
    n, k = w.shape
    m = x.shape[0]
    y = np.empty((m, n), np.float32)
    sec = ctypes.c_double()
    _check(_load().ref_bitlinear_time_forward(w, n, k, x, m, int(exact_linear), int(reps), y,
                                              ctypes.byref(sec)), "bitlinear_time_forward")
    return sec.value, y


def mamba2_faithful_forward(p: dict, u, packed: bool = True):
    """Mamba2SSD::forward on the faithful path (src/mamba2.cpp:2360-2681) with the caller's
    parameters (Mamba2Block's dict: w_x, w_z, w_B, w_C, w_dt, dt_bias, w_out, conv_w, conv_b,
    a_log, d_skip, norm_w; H, P, N, G).  packed: x / z / out_proj on the packed ternary path,
    B / C / dt float.  u [batch, seq, d] -> out [batch, seq, d]."""
    lib = _load()
    fn = lib.ref_mamba2_faithful_forward
    fn.restype = _i
    fn.argtypes = [_i] * 6 + [_f32p] * 12 + [_i, _f32p, _i, _i, _f32p]
    u = _f32(u)
    b, s, d = u.shape
    H, P, N, G = (int(p[k]) for k in ("H", "P", "N", "G"))
    inner = H * P
    out = np.empty_like(u)
    args = [_f32(p[k]) for k in ("w_x", "w_z", "w_B", "w_C", "w_dt", "dt_bias", "w_out",
                                 "conv_w", "conv_b", "a_log", "d_skip", "norm_w")]
    _check(fn(d, N, inner // d, P, G, p["conv_w"].shape[1], *args, int(packed), u, b, s, out),
           "mamba2_faithful_forward")
    return out
