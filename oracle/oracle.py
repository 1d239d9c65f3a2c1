"""numpy front end of the C oracle (oracle/nsos_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as
the checker and by bench.py's cpu_baseline leg.  The shipped package
(reimagined_amd) never imports this module.

Each wrapper names the reference function it restates; the C file carries the
file:line citations.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libnsos_ref.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float


def build() -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is mounted)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    if os.path.isdir("/root/reference/OXN/nsos/src"):
        subprocess.run(["make", "-s", "-C", _HERE, "ref"], check=True)


def _load() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_absmean": (_f, [_f32p, _i64]),
        "orc_weight_scale": (_f, [_f32p, _i64]),
        "orc_ternary_codes": (None, [_f32p, _i64, _f, _i8p]),
        "orc_pack_codes": (None, [_i8p, _i64, _u8p]),
        "orc_unpack_codes": (None, [_u8p, _i64, _i8p]),
        "orc_find_reserved_code": (_i64, [_u8p, _i64]),
        "orc_row_sums": (None, [_i8p, _i, _i, _i32p]),
        "orc_q_max": (_f, [_i]),
        "orc_rmsnorm": (None, [_f32p, _i, _i, _f, _f32p]),
        "orc_quantize_act": (None, [_f32p, _i, _i, _i, _i8p, _f32p]),
        "orc_gemm_i8": (None, [_i8p, _i8p, _i, _i, _i, _i32p]),
        "orc_dequant": (None, [_i32p, _f32p, _f, _vp, _vp, _i, _i, _f32p]),
        "orc_bitlinear_forward": (None, [_f32p, _i, _i, _i, _u8p, _f, _i, _i, _vp, _vp,
                                         _f32p, _vp, _vp, _vp]),
        "orc_silu": (_f, [_f]),
        "orc_softplus": (_f, [_f]),
        "orc_squared_relu": (None, [_f32p, _i64, _f32p]),
        "orc_decay_terms": (None, [_f, _f, ctypes.POINTER(_f), ctypes.POINTER(_f)]),
        "orc_conv1d_causal": (None, [_f32p, _f32p, _vp, _i32p, _i, _i, _i, _i, _f32p]),
        "orc_selective_scan": (None, [_f32p, _f32p, _f32p, _i, _f32p, _f32p, _f32p, _vp,
                                      _i32p, _i, _i, _i, _i, _i, _vp, _f32p, _vp, _i]),
        "orc_scan_step": (None, [_f32p, _f32p, _f32p, _i, _f32p, _f32p, _f32p, _vp,
                                 _i, _i, _i, _i, _i, _f32p, _f32p, _i]),
        "orc_conv_step": (None, [_f32p, _i, _i, _f32p, _vp, _i, _vp, _i, _f32p]),
        "orc_rmsnorm_gated": (None, [_f32p, _vp, _vp, _i, _i, _f, _f32p]),
        "orc_qat_fake_quant_ternary": (None, [_f32p, _i64, _f, _f32p]),
        "orc_qat_fake_quant_ternary_absmean": (_f, [_f32p, _i64, _f32p]),
        "orc_qat_fake_quant_activations": (None, [_f32p, _i, _i, _i, _f32p]),
        "orc_qat_ste_clip": (None, [_f32p, _f32p, _i64, _f]),
        "orc_rmsnorm_backward": (None, [_f32p, _f32p, _f32p, _i, _i, _f, _f32p]),
        "orc_linear_f32": (None, [_f32p, _i, _i, _i, _f32p, _i, _vp, _vp, _f32p]),
        "orc_bitlinear_ste_backward": (None, [_f32p, _i8p, _f32p, _f32p, _i8p, _f, _i, _i, _i,
                                              _i, _vp, _f32p, _f32p, _f32p, _vp, _vp]),
        "orc_softmax_rows": (None, [_f32p, _i, _i, _f32p]),
        "orc_topk_mask": (None, [_f32p, _i, _i, _i, _vp]),
        "orc_moe_dispatch": (None, [_f32p, _i, _i, _i, _i32p, _i32p, _i32p]),
        "orc_zero_invalid_rows": (None, [_f32p, _i32p, _u8p, _i, _i, _i]),
        "orc_expert_loads": (None, [_f32p, _vp, _i, _i, _f32p]),
        "orc_moe_dispatch_sel": (None, [_i32p, _i, _i, _i, _i32p, _i32p, _i32p]),
        "orc_moe_combine": (None, [_f32p, _i32p, _i32p, _f32p, _i, _i, _i, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = _load()


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---- weights -------------------------------------------------------------

def absmean(w) -> float:
    """tensor_abs_mean (OXN/nsos/src/tensor.cpp:2100-2107)."""
    w = _f32(w)
    return float(_lib.orc_absmean(w.ravel(), w.size))


def weight_scale(w) -> float:
    """BitLinear::pack_weights weight_scale = absmean + 1e-8f."""
    w = _f32(w)
    return float(np.float32(_lib.orc_weight_scale(w.ravel(), w.size)))


def ternary_codes(w, ws: float | None = None) -> np.ndarray:
    """BitLinear::quantize_weights -> int8 codes in {-1,0,+1}, same shape as w."""
    w = _f32(w)
    if ws is None:
        ws = weight_scale(w)
    out = np.empty(w.shape, np.int8)
    _lib.orc_ternary_codes(w.ravel(), w.size, ws, out.ravel())
    return out


def pack_codes(codes) -> np.ndarray:
    """pack_weights_microsoft_style -> uint8 bytes, ceil(n/4) long."""
    codes = np.ascontiguousarray(codes, dtype=np.int8).ravel()
    out = np.zeros((codes.size + 3) // 4, np.uint8)
    _lib.orc_pack_codes(codes, codes.size, out)
    return out


def unpack_codes(packed, n: int) -> np.ndarray:
    """unpack_weights_microsoft_style_to_i8 (reserved code 3 -> 0)."""
    packed = np.ascontiguousarray(packed).view(np.uint8).ravel()
    out = np.empty(n, np.int8)
    _lib.orc_unpack_codes(packed, n, out)
    return out


def find_reserved_code(packed, n: int) -> int:
    packed = np.ascontiguousarray(packed).view(np.uint8).ravel()
    return int(_lib.orc_find_reserved_code(packed, n))


def pack_weights(w):
    """BitLinear::pack_weights for a float [N, K] matrix.

    Returns (packed uint32 [N*K/16] for K % 16 == 0, weight_scale, codes int8 [N,K]).
    """
    w = _f32(w)
    ws = weight_scale(w)
    codes = ternary_codes(w, ws)
    packed = pack_codes(codes)
    pad = (-packed.size) % 4
    if pad:
        packed = np.concatenate([packed, np.zeros(pad, np.uint8)])
    return packed.view(np.uint32), ws, codes


def row_sums(w_codes) -> np.ndarray:
    w_codes = np.ascontiguousarray(w_codes, dtype=np.int8)
    out = np.empty(w_codes.shape[0], np.int32)
    _lib.orc_row_sums(w_codes, w_codes.shape[0], w_codes.shape[1], out)
    return out


# ---- activations / GEMM -------------------------------------------------

def q_max(bits: int) -> float:
    return float(_lib.orc_q_max(bits))


def rmsnorm(x, eps: float = 1e-6) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    _lib.orc_rmsnorm(x, x.shape[0], x.shape[1], eps, out)
    return out


def quantize_act(x, bits: int = 8):
    """quantize_activations_bitnet + the GEMM's int8 clamp -> (int8 [M,K], act_scale [M])."""
    x = _f32(x)
    m, k = x.shape
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    _lib.orc_quantize_act(x, m, k, bits, q, s)
    return q, s


def gemm_i8(q, w_codes) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    w_codes = np.ascontiguousarray(w_codes, dtype=np.int8)
    m, k = q.shape
    n = w_codes.shape[0]
    acc = np.empty((m, n), np.int32)
    _lib.orc_gemm_i8(q, w_codes, m, k, n, acc)
    return acc


def dequant(acc, act_scale, ws: float, magnitude=None, bias=None) -> np.ndarray:
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    act_scale = _f32(act_scale)
    mag = None if magnitude is None else _f32(magnitude)
    b = None if bias is None else _f32(bias)
    m, n = acc.shape
    y = np.empty((m, n), np.float32)
    _lib.orc_dequant(acc, act_scale, ws, _ptr(mag), _ptr(b), m, n, y)
    return y


def bitlinear_forward(x, packed, ws: float, n_out: int, bits: int = 8, rms_input: bool = False,
                      magnitude=None, bias=None, want_intermediates: bool = False):
    """BitLinear::forward on the CPU packed path (optionally RMS_PERI)."""
    x = _f32(x)
    m, k = x.shape
    packed = np.ascontiguousarray(packed).view(np.uint8).ravel()
    mag = None if magnitude is None else _f32(magnitude)
    b = None if bias is None else _f32(bias)
    y = np.empty((m, n_out), np.float32)
    q = np.empty((m, k), np.int8)
    s = np.empty(m, np.float32)
    acc = np.empty((m, n_out), np.int32)
    _lib.orc_bitlinear_forward(x, m, k, n_out, packed, ws, bits, int(rms_input), _ptr(mag),
                               _ptr(b), y, _ptr(q), _ptr(s), _ptr(acc))
    if want_intermediates:
        return y, q, s, acc
    return y


# ---- elementwise ------------------------------------------------------------

def silu(v: float) -> float:
    return float(_lib.orc_silu(v))


def softplus(v: float) -> float:
    return float(_lib.orc_softplus(v))


def squared_relu(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty_like(x)
    _lib.orc_squared_relu(x.ravel(), x.size, out.ravel())
    return out


def silu_array(x) -> np.ndarray:
    x = _f32(x)
    f = np.vectorize(lambda v: np.float32(_lib.orc_silu(float(v))), otypes=[np.float32])
    return f(x)


# ---- Mamba -----------------------------------------------------------------

def decay_terms(dt_raw: float, a_log: float):
    d = _f()
    k = _f()
    _lib.orc_decay_terms(dt_raw, a_log, ctypes.byref(d), ctypes.byref(k))
    return d.value, k.value


def conv1d_causal(x, weight, cu_seqlens, bias=None, silu_act: bool = True) -> np.ndarray:
    x = _f32(x)
    weight = _f32(weight)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    b = None if bias is None else _f32(bias)
    out = np.zeros_like(x)
    _lib.orc_conv1d_causal(x, weight, _ptr(b), cu, cu.size - 1, x.shape[1], weight.shape[1],
                           int(silu_act), out)
    return out


def conv_step(x, weight, bias, ring, silu_act: bool = True):
    """Decode conv ring step -> (out [R, C], new ring [R, W-1, C]); `ring` is not touched."""
    x = _f32(x)
    weight = _f32(weight)
    b = None if bias is None else _f32(bias)
    rg = None if ring is None else _f32(ring).copy()
    out = np.empty_like(x)
    _lib.orc_conv_step(x, x.shape[0], x.shape[1], weight, _ptr(b), weight.shape[1], _ptr(rg),
                       int(silu_act), out)
    return out, rg


def rmsnorm_gated(y, z=None, gamma=None, eps: float = 1e-5) -> np.ndarray:
    """RMSNorm(y * silu(z)) * gamma (z None: rmsnorm(y) * gamma; gamma None: unit)."""
    y = _f32(y)
    zz = None if z is None else _f32(z)
    g = None if gamma is None else _f32(gamma)
    out = np.empty_like(y)
    _lib.orc_rmsnorm_gated(y, _ptr(zz), _ptr(g), y.shape[0], y.shape[1], eps, out)
    return out


def selective_scan(x, dt, a_log, B, C, Dskip, z, cu_seqlens, H, P, N, G,
                   initial_state=None, gate_silu: bool = True):
    """Faithful recurrence over a packed ragged batch -> (y [T, H*P], final [S, H*P, N])."""
    x = _f32(x)
    dt = _f32(dt)
    a_log = _f32(a_log)
    B = _f32(B)
    C = _f32(C)
    Dskip = _f32(Dskip)
    zz = None if z is None else _f32(z)
    cu = np.ascontiguousarray(cu_seqlens, dtype=np.int32)
    s = cu.size - 1
    a_per_state = int(a_log.size == H * N and N > 1)
    h0 = None if initial_state is None else _f32(initial_state)
    y = np.empty_like(x)
    fin = np.empty((s, H * P, N), np.float32)
    _lib.orc_selective_scan(x, dt, a_log.ravel(), a_per_state, B, C, Dskip, _ptr(zz), cu, s,
                            H, P, N, G, _ptr(h0), y, _ptr(fin), int(gate_silu and z is not None))
    return y, fin


def scan_step(x, dt, a_log, B, C, Dskip, z, state, H, P, N, G, gate_silu: bool = True):
    """Decode step; returns (y [R, D], new_state [R, D, N]) without touching `state`."""
    x = _f32(x)
    dt = _f32(dt)
    a_log = _f32(a_log)
    st = _f32(state).copy()
    zz = None if z is None else _f32(z)
    y = np.empty_like(x)
    a_per_state = int(a_log.size == H * N and N > 1)
    _lib.orc_scan_step(x, dt, a_log.ravel(), a_per_state, _f32(B), _f32(C), _f32(Dskip),
                       _ptr(zz), x.shape[0], H, P, N, G, st, y,
                       int(gate_silu and z is not None))
    return y, st


# ---- MoE ---------------------------------------------------------------------

def softmax_rows(logits) -> np.ndarray:
    logits = _f32(logits)
    out = np.empty_like(logits)
    _lib.orc_softmax_rows(logits, logits.shape[0], logits.shape[1], out)
    return out


def topk_mask(probs, k: int, valid=None):
    """-> (masked renormalised weights, selected expert ids [rows, k] in rank order).
    valid: the 0/1 padding mask of MoERouter::forward(x, valid_rows); padding rows get
    zero weights and selections -1."""
    w = _f32(probs).copy()
    rows, e = w.shape
    sel = np.empty((rows, k), np.int32)
    _lib.orc_topk_mask(w, rows, e, k, _ptr(sel))
    if valid is not None:
        v = np.ascontiguousarray(valid, dtype=np.uint8)
        _lib.orc_zero_invalid_rows(w, sel, v, rows, e, k)
    return w, sel


def moe_dispatch(weights, k: int):
    """-> (counts [E], offsets [E+1], perm [rows*k]) expert-major, rows ascending."""
    w = _f32(weights)
    rows, e = w.shape
    counts = np.empty(e, np.int32)
    offsets = np.empty(e + 1, np.int32)
    perm = np.empty(rows * k, np.int32)
    _lib.orc_moe_dispatch(w, rows, e, k, counts, offsets, perm)
    return counts, offsets, perm


def moe_dispatch_sel(selected, experts: int):
    """The dispatch of a selection [rows, k] (-1 = no expert) -> (counts, offsets, perm);
    perm holds offsets[E] rows (the rest of its rows * k entries are -1)."""
    sel = np.ascontiguousarray(selected, dtype=np.int32)
    rows, k = sel.shape
    counts = np.empty(experts, np.int32)
    offsets = np.empty(experts + 1, np.int32)
    perm = np.full(rows * k, -1, np.int32)
    _lib.orc_moe_dispatch_sel(sel, rows, experts, k, counts, offsets, perm)
    return counts, offsets, perm


def expert_loads(weights, valid=None) -> np.ndarray:
    """MoERouter::forward's expert_loads: per-expert in-order sums of the weights over
    the valid rows."""
    w = _f32(weights)
    rows, e = w.shape
    loads = np.empty(e, np.float32)
    v = None if valid is None else np.ascontiguousarray(valid, dtype=np.uint8)
    _lib.orc_expert_loads(w, None if v is None else v.ctypes.data_as(_vp), rows, e, loads)
    return loads


def moe_combine(expert_out, perm, offsets, weights) -> np.ndarray:
    expert_out = _f32(expert_out)
    perm = np.ascontiguousarray(perm, dtype=np.int32)
    offsets = np.ascontiguousarray(offsets, dtype=np.int32)
    w = _f32(weights)
    rows, e = w.shape
    out = np.empty((rows, expert_out.shape[1]), np.float32)
    _lib.orc_moe_combine(expert_out, perm, offsets, w, rows, e, expert_out.shape[1], out)
    return out


# ---- float (quantization-sensitive) path and the packed STE backward -----------

def rmsnorm_backward(x, grad, x_norm, eps: float = 1e-6) -> np.ndarray:
    """Tensor::rmsnorm_backward (src/tensor.cpp:3997-4056)."""
    x, grad, x_norm = _f32(x), _f32(grad), _f32(x_norm)
    out = np.empty_like(x)
    _lib.orc_rmsnorm_backward(x, grad, x_norm, x.shape[0], x.shape[1], eps, out)
    return out


def linear_f32(x, w, rms_input: bool = False, magnitude=None, bias=None) -> np.ndarray:
    """BitLinear's float reference path (src/bitlinear.cpp:465-518): [rmsnorm] x @ W^T
    (double accumulation), then *magnitude, +bias."""
    x, w = _f32(x), _f32(w)
    m, k = x.shape
    n = w.shape[0]
    mag = None if magnitude is None else _f32(magnitude)
    b = None if bias is None else _f32(bias)
    y = np.empty((m, n), np.float32)
    _lib.orc_linear_f32(x, m, k, n, w, int(rms_input), _ptr(mag), _ptr(b), y)
    return y


def bitlinear_ste_backward(x, w, grad, rms_input: bool = True, magnitude=None,
                           use_bias: bool = False, bits: int = 8) -> dict:
    """BitLinear forward (packed path) then its STE backward (src/bitlinear.cpp:1191-1357).

    Returns dx, dW, dmag (with magnitude), dbias (use_bias), plus the forward's q / as /
    codes / weight_scale."""
    x, w, grad = _f32(x), _f32(w), _f32(grad)
    m, k = x.shape
    n = w.shape[0]
    packed, ws, codes = pack_weights(w)
    src = rmsnorm(x) if rms_input else x
    q, s = quantize_act(src, bits)
    mag = None if magnitude is None else _f32(magnitude)
    out = {"dx": np.empty((m, k), np.float32), "dW": np.empty((n, k), np.float32),
           "q": q, "act_scale": s, "codes": codes, "weight_scale": ws, "packed": packed}
    dmag = np.empty(n, np.float32) if mag is not None else None
    dbias = np.empty(n, np.float32) if use_bias else None
    _lib.orc_bitlinear_ste_backward(x, q, s, w, codes, ws, m, k, n, int(rms_input), _ptr(mag),
                                    grad, out["dx"], out["dW"], _ptr(dmag), _ptr(dbias))
    if dmag is not None:
        out["dmag"] = dmag
    if dbias is not None:
        out["dbias"] = dbias
    return out


# ---- reference build (oracle/_ref), present only where the reference is --------

def ref_available() -> bool:
    return os.path.exists(_REF_PATH)


def ref_quantize_rows(x, bits: int = 8):
    """The reference's own AVX2 row quantizer -> (float codes [M,K], act_scale [M])."""
    lib = ctypes.CDLL(_REF_PATH)
    lib.ref_quantize_rows.restype = None
    lib.ref_quantize_rows.argtypes = [_f32p, _i, _i, _i, _f32p, _f32p]
    x = _f32(x)
    m, k = x.shape
    codes = np.empty((m, k), np.float32)
    scales = np.empty(m, np.float32)
    lib.ref_quantize_rows(x, m, k, bits, codes, scales)
    return codes, scales


def ref_row_sum_i8(row) -> int:
    lib = ctypes.CDLL(_REF_PATH)
    lib.ref_row_sum_i8.restype = ctypes.c_int32
    lib.ref_row_sum_i8.argtypes = [_i8p, _i]
    row = np.ascontiguousarray(row, dtype=np.int8)
    return int(lib.ref_row_sum_i8(row, row.size))


# ---- quantization-aware training -----------------------------------------------

def qat_fake_quant_ternary(w, scale):
    """qat_fake_quant_ternary (src/bitnet_gpu_dispatch.cpp:193-217)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(w)
    _lib.orc_qat_fake_quant_ternary(w.ravel(), w.size, float(scale), out.ravel())
    return out


def qat_fake_quant_ternary_absmean(w):
    """qat_fake_quant_ternary_absmean (src/bitnet_gpu_dispatch.cpp:219-245) -> (out, scale)."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(w)
    scale = _lib.orc_qat_fake_quant_ternary_absmean(w.ravel(), w.size, out.ravel())
    return out, np.float32(scale)


def qat_fake_quant_activations(x, bits=8):
    """qat_fake_quant_activations (src/bitnet_gpu_dispatch.cpp:247-282), rows = last dim."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    out = np.empty_like(x)
    _lib.orc_qat_fake_quant_activations(x.ravel(), x.size // k, k, int(bits), out.ravel())
    return out


def qat_ste_clip(dW, w, scale):
    """qat_ste_clip_weight_grad (src/bitnet_gpu_dispatch.cpp:284-308) on a copy of dW."""
    out = np.array(dW, dtype=np.float32, copy=True)
    w = np.ascontiguousarray(w, dtype=np.float32)
    _lib.orc_qat_ste_clip(out.ravel(), w.ravel(), w.size, float(scale))
    return out
