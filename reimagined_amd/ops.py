"""Host-side operators over the nsosx C ABI (torch supplies device memory and streams).

Each function mirrors the reference operator it replaces (OXN/nsos/ of
vitorGgC569/reimagined): argument meaning, shapes and error behaviour
(ValueError for rejected shapes, as the reference's std::invalid_argument).
All work is enqueued on torch's current stream without synchronising.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from ._lib import NsosxError, call, lib

F32, BF16 = 0, 1
_DT = {torch.float32: F32, torch.bfloat16: BF16}


def _dt(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}: float32 or bfloat16") from None


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _dev(t: torch.Tensor, name: str, dtype=None) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    return t


def _opt(t, name: str, dtype=torch.float32):
    return None if t is None else _dev(t, name, dtype)


# ---- weights -------------------------------------------------------------------

def pack_ternary(w) -> tuple[np.ndarray, float]:
    """BitLinear::pack_weights (src/bitlinear.cpp:152-193) on the host.

    w: float [N, K] (numpy or CPU tensor).  Returns (packed uint32 [N*K/16], weight_scale).
    """
    w = np.ascontiguousarray(w.numpy() if isinstance(w, torch.Tensor) else w, dtype=np.float32)
    if w.ndim != 2:
        raise ValueError("pack_ternary expects a 2-D [N, K] matrix")
    n, k = w.shape
    packed = np.zeros(n * k // 16 if k % 16 == 0 else 0, np.uint32)
    ws = ctypes.c_float()
    call("nsosx_pack_ternary", w.ctypes.data_as(ctypes.c_void_p), n, k,
         packed.ctypes.data_as(ctypes.c_void_p), ctypes.byref(ws))
    return packed, float(ws.value)


def unpack_ternary(packed, n: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint32)
    out = np.empty(n, np.int8)
    call("nsosx_unpack_ternary", packed.ctypes.data_as(ctypes.c_void_p), n,
         out.ctypes.data_as(ctypes.c_void_p))
    return out


def find_reserved_code(packed: torch.Tensor, n_codes: int) -> int:
    """Device import check (src/bitlinear.cpp:876-885): index of the first code 3, or -1."""
    _dev(packed, "packed")
    out = torch.empty(1, dtype=torch.int64, device=packed.device)
    call("nsosx_find_reserved_code", _p(packed), n_codes, _p(out), _stream())
    return int(out.item())


def weight_row_sums(packed: torch.Tensor, n: int, k: int) -> torch.Tensor:
    """compute_weight_row_sums (src/bitlinear.cpp:36-73) on the device -> int32 [N]."""
    _dev(packed, "packed")
    if k <= 0 or k % 16 or packed.numel() != n * k // 16:
        raise ValueError("weight_row_sums: packed must hold N*K/16 words with K % 16 == 0")
    out = torch.empty(n, dtype=torch.int32, device=packed.device)
    call("nsosx_weight_row_sums", _p(packed), n, k, _p(out), _stream())
    return out


# ---- BitLinear ------------------------------------------------------------------

def quantize_activations_bitnet(x: torch.Tensor, bits: int = 8, rms_input: bool = False):
    """quantize_activations_bitnet (+ RMS_PERI) -> (q int8 [M,K], act_scale f32 [M])."""
    _dev(x, "x")
    m, k = x.shape
    q = torch.empty((m, k), dtype=torch.int8, device=x.device)
    s = torch.empty(m, dtype=torch.float32, device=x.device)
    ws = torch.empty(m, dtype=torch.float32, device=x.device) if rms_input else None
    call("nsosx_quantize_act_i8", _p(x), _dt(x), m, k, bits, int(rms_input), _p(q), _p(s), _p(ws),
         _stream())
    return q, s


def ternary_gemm(q: torch.Tensor, act_scale: torch.Tensor, packed: torch.Tensor, ws: float,
                 n_out: int, magnitude=None, bias=None, out_dtype=torch.float32,
                 want_acc: bool = False, path: int | None = None, want_y: bool = True):
    """gemm_158bit_i8 integer core + affine (src/bitnet_adapter_avx2.cpp:52-158).

    Returns y [M, N] (or (y, acc int32 [M, N]) with want_acc).
    """
    _dev(q, "q", torch.int8)
    _dev(act_scale, "act_scale", torch.float32)
    _dev(packed, "packed")
    if packed.dtype not in (torch.int32, torch.uint32):
        raise ValueError("packed must hold 32-bit words")
    _opt(magnitude, "magnitude")
    _opt(bias, "bias")
    m, k = q.shape
    y = torch.empty((m, n_out), dtype=out_dtype, device=q.device) if want_y else None
    acc = torch.empty((m, n_out), dtype=torch.int32, device=q.device) if want_acc else None
    ydt = _DT[out_dtype]
    if path is None:
        call("nsosx_ternary_gemm", _p(q), _p(act_scale), _p(packed), ws, m, k, n_out,
             _p(magnitude), _p(bias), _p(y), ydt, _p(acc), _stream())
    else:
        call("nsosx_ternary_gemm_path", _p(q), _p(act_scale), _p(packed), ws, m, k, n_out,
             _p(magnitude), _p(bias), _p(y), ydt, _p(acc), path, _stream())
    if want_acc:
        return y, acc
    return y


def skinny_shape(m: int, k: int, n: int) -> bool:
    """The shapes the skinny MFMA decode kernel takes (the library's skinny_ok): 2 <= m <=
    32, k in {1024, 2048, 4096}, ceil(m / 16) * k <= 4096, m * n * 4 < 2^31."""
    return (2 <= m <= 32 and k in (1024, 2048, 4096) and ((m + 15) // 16) * k <= 4096
            and m * n * 4 < 2**31)


def pack_mfma_layout(packed: torch.Tensor) -> torch.Tensor:
    """The prefill GEMM's weight layout (a device repack of reference-layout words)."""
    _dev(packed, "packed")
    out = torch.empty_like(packed)
    call("nsosx_pack_mfma_layout", _p(packed), packed.numel(), _p(out), _stream())
    return out


def ternary_gemm_mfma(q: torch.Tensor, act_scale: torch.Tensor, packed_mfma: torch.Tensor,
                      ws: float, n_out: int, magnitude=None, bias=None,
                      out_dtype=torch.float32, want_acc: bool = False):
    """ternary_gemm on MFMA-layout weights (the prefill MFMA GEMM, K % 128 == 0)."""
    _dev(q, "q", torch.int8)
    _dev(act_scale, "act_scale", torch.float32)
    _dev(packed_mfma, "packed_mfma")
    _opt(magnitude, "magnitude")
    _opt(bias, "bias")
    m, k = q.shape
    y = torch.empty((m, n_out), dtype=out_dtype, device=q.device)
    acc = torch.empty((m, n_out), dtype=torch.int32, device=q.device) if want_acc else None
    call("nsosx_ternary_gemm_mfma", _p(q), _p(act_scale), _p(packed_mfma), ws, m, k, n_out,
         _p(magnitude), _p(bias), _p(y), _DT[out_dtype], _p(acc), _stream())
    return (y, acc) if want_acc else y


def bitnet_gemm_158bit_gpu(x: torch.Tensor, packed: torch.Tensor, weight_scale: float, M: int,
                           K: int, N: int, precision_bits: int = 8, magnitude=None, bias=None,
                           rms_input: bool = False, out_dtype=torch.float32) -> torch.Tensor:
    """bitnet_gemm_158bit_gpu (include/bitnet_gpu_dispatch.h:46-51): quantize + ternary GEMM."""
    _dev(x, "x")
    _dev(packed, "packed")
    if x.numel() != M * K:
        raise ValueError("bitnet_gemm_158bit_gpu: x does not hold M*K elements")
    qw = torch.empty((M, K), dtype=torch.int8, device=x.device)
    sw = torch.empty(M, dtype=torch.float32, device=x.device)
    rw = torch.empty(M, dtype=torch.float32, device=x.device) if rms_input else None
    y = torch.empty((M, N), dtype=out_dtype, device=x.device)
    call("nsosx_bitlinear_forward", _p(x), _dt(x), _p(packed), weight_scale, M, K, N,
         precision_bits, int(rms_input), _p(magnitude), _p(bias), _p(y), _DT[out_dtype], _p(qw),
         _p(sw), _p(rw), _stream())
    return y


def linear_f32(x: torch.Tensor, w: torch.Tensor, rms_input: bool = False, magnitude=None,
               bias=None, out_dtype=torch.float32, out=None) -> torch.Tensor:
    """BitLinear's float reference path for quantization-sensitive layers
    (src/bitlinear.cpp:465-518): [rmsnorm] x @ w^T, then * magnitude, then + bias."""
    _dev(x, "x")
    _dev(w, "w", torch.float32)
    _opt(magnitude, "magnitude")
    _opt(bias, "bias")
    if x.dim() != 2 or w.dim() != 2 or w.shape[1] != x.shape[1]:
        raise ValueError("linear_f32: x [M, K] and w [N, K] must agree in K")
    m, k = x.shape
    n = w.shape[0]
    for name, v in (("magnitude", magnitude), ("bias", bias)):
        if v is not None and v.numel() != n:
            raise ValueError(f"linear_f32: {name} must hold N = {n} values")
    if out is None:
        out = torch.empty((m, n), dtype=out_dtype, device=x.device)
    elif tuple(out.shape) != (m, n) or not out.is_contiguous():
        raise ValueError("linear_f32: out must be a contiguous [M, N] tensor")
    rw = torch.empty(m, dtype=torch.float32, device=x.device) if rms_input else None
    call("nsosx_linear_f32", _p(x), _dt(x), m, k, _p(w), n, int(rms_input), _p(magnitude),
         _p(bias), _p(out), _dt(out), _p(rw), _stream())
    return out


def bitlinear_ste_backward(x, q, act_scale, w_latent, packed, weight_scale: float, grad,
                           rms_input: bool = True, magnitude=None, want_dbias: bool = False,
                           want_dmag: bool = True) -> dict:
    """BitLinear::backward on the packed path (src/bitlinear.cpp:1191-1357) from what the
    forward saved: x [M, K], its int8 codes q and act_scale, the latent weights [N, K] and
    their packed ternary; grad [M, N].  Returns dx, dW (+ dmag, dbias)."""
    for name, v, dt in (("q", q, torch.int8), ("act_scale", act_scale, torch.float32),
                        ("w_latent", w_latent, torch.float32), ("grad", grad, torch.float32)):
        _dev(v, name, dt)
    _dev(packed, "packed")
    _opt(magnitude, "magnitude")
    m, k = q.shape
    n = w_latent.shape[0]
    if tuple(grad.shape) != (m, n) or tuple(w_latent.shape) != (n, k) or \
            act_scale.numel() != m or packed.numel() != n * k // 16:
        raise ValueError("bitlinear_ste_backward: inconsistent shapes")
    if rms_input:
        _dev(x, "x")
        if tuple(x.shape) != (m, k):
            raise ValueError("bitlinear_ste_backward: x must be [M, K]")
    dev = q.device
    out = {"dx": torch.empty((m, k), dtype=torch.float32, device=dev),
           "dW": torch.empty((n, k), dtype=torch.float32, device=dev)}
    if magnitude is not None and want_dmag:
        out["dmag"] = torch.empty(n, dtype=torch.float32, device=dev)
    if want_dbias:
        out["dbias"] = torch.empty(n, dtype=torch.float32, device=dev)
    nbytes = int(lib().nsosx_bitlinear_ste_backward_workspace(m, k, n, int(rms_input)))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    call("nsosx_bitlinear_ste_backward", _p(x) if rms_input else None,
         _dt(x) if rms_input else F32, _p(q), _p(act_scale), _p(w_latent), _p(packed),
         float(weight_scale), m, k, n, int(rms_input), _p(magnitude), _p(grad), _p(out["dx"]),
         _p(out["dW"]), _p(out.get("dmag")), _p(out.get("dbias")), _p(ws), _stream())
    return out


class LinearViewArray:
    """Device array of nsosx_linear_view descriptors (GpuLinearView's C shape).

    Borrows the tensors it points at; keeps Python references so they outlive it.
    """

    class _View(ctypes.Structure):
        _fields_ = [("packed", ctypes.c_void_p), ("magnitude", ctypes.c_void_p),
                    ("bias", ctypes.c_void_p), ("inputs", ctypes.c_int),
                    ("outputs", ctypes.c_int), ("weight_scale", ctypes.c_float)]

    def __init__(self, entries, device):
        self._keep = []
        arr = (self._View * len(entries))()
        for i, (packed, ws, inputs, outputs, mag, bias) in enumerate(entries):
            self._keep += [packed, mag, bias]
            arr[i].packed = packed.data_ptr()
            arr[i].magnitude = None if mag is None else mag.data_ptr()
            arr[i].bias = None if bias is None else bias.data_ptr()
            arr[i].inputs = inputs
            arr[i].outputs = outputs
            arr[i].weight_scale = ws
        raw = bytes(arr)
        host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
        self.tensor = host.to(device)
        self.count = len(entries)

    @property
    def ptr(self):
        return ctypes.c_void_p(self.tensor.data_ptr())


class DecodeViewArray:
    """Device array of nsosx_decode_view descriptors (GpuLinearView, include/gpu_linear_view.h:8-25):
    entries are dicts with either `packed` (int32 words) + `weight_scale` + `bits`, or `weight`
    (f32 [outputs, inputs]); `inputs`, `outputs`, optional `magnitude`, `bias`, `rms_input`."""

    class _View(ctypes.Structure):
        _fields_ = [("weight", ctypes.c_void_p), ("packed", ctypes.c_void_p),
                    ("magnitude", ctypes.c_void_p), ("bias", ctypes.c_void_p),
                    ("inputs", ctypes.c_int), ("outputs", ctypes.c_int),
                    ("activation_bits", ctypes.c_int), ("rms_input", ctypes.c_int),
                    ("weight_scale", ctypes.c_float)]

    def __init__(self, entries, device):
        self._keep = []
        arr = (self._View * len(entries))()
        for i, e in enumerate(entries):
            ptr = lambda t: None if t is None else t.data_ptr()
            for k in ("weight", "packed", "magnitude", "bias"):
                if e.get(k) is not None:
                    self._keep.append(e[k])
            arr[i].weight = ptr(e.get("weight"))
            arr[i].packed = ptr(e.get("packed"))
            arr[i].magnitude = ptr(e.get("magnitude"))
            arr[i].bias = ptr(e.get("bias"))
            arr[i].inputs = int(e["inputs"])
            arr[i].outputs = int(e["outputs"])
            arr[i].activation_bits = int(e.get("bits", 0 if e.get("packed") is None else 8))
            arr[i].rms_input = int(bool(e.get("rms_input", False)))
            arr[i].weight_scale = float(e.get("weight_scale", 1.0))
        self.tensor = torch.frombuffer(bytearray(bytes(arr)), dtype=torch.uint8).to(device)
        self.count = len(entries)
        self.max_outputs = max(int(e["outputs"]) for e in entries)

    @property
    def ptr(self):
        return ctypes.c_void_p(self.tensor.data_ptr())


def grouped_decode_projections(views: DecodeViewArray, x: torch.Tensor, out_dtype=None,
                               out=None) -> torch.Tensor:
    """GpuProjectionGroup::forward (src/gpu_projection_group.cpp:12-49): one input row
    through every view -> [views, max outputs] (row g holds view g's outputs first)."""
    _dev(x, "x")
    if x.dim() != 1 and not (x.dim() == 2 and x.shape[0] == 1):
        raise ValueError("grouped_decode_projections: x must be one row")
    odt = out_dtype or x.dtype
    if out is None:
        out = torch.empty((views.count, views.max_outputs), dtype=odt, device=x.device)
    elif tuple(out.shape) != (views.count, views.max_outputs) or not out.is_contiguous():
        raise ValueError("grouped_decode_projections: out must be [views, max outputs]")
    call("nsosx_grouped_decode_projections", views.ptr, views.count, _p(x), _dt(x), _p(out),
         views.max_outputs, _dt(out), _stream())
    return out


def grouped_gemv(views: LinearViewArray, q: torch.Tensor, act_scale: torch.Tensor, n_out: int,
                 out_dtype=torch.bfloat16) -> torch.Tensor:
    """Grouped decode projections (include/cuda/kernels.cuh:27-29).

    q: int8 [G, M, K]; act_scale [G, M]; returns y [G, M, n_out].
    """
    g, m, k = q.shape
    y = torch.empty((g, m, n_out), dtype=out_dtype, device=q.device)
    call("nsosx_grouped_gemv", views.ptr, g, _p(q), m * k, _p(act_scale), m, m, _p(y), m * n_out,
         _DT[out_dtype], _stream())
    return y


# ---- Mamba ----------------------------------------------------------------------

def _shape(t, want: tuple, name: str, fn: str) -> None:
    if t is not None and tuple(t.shape) != tuple(want):
        raise ValueError(f"{fn}: {name} must have shape {tuple(want)}, got {tuple(t.shape)}")


def _check_scan_shapes(fn, x, dt, a_log, B, C, D, z, H, P, N, G, t_rows=None):
    """Host-side shape checks of the scan inputs: the C ABI takes raw pointers, so an
    undersized buffer would be read or written out of bounds on the device."""
    if min(H, P, N, G) <= 0 or H % G:
        raise ValueError(f"{fn}: need positive H, P, N, G with G dividing H")
    if x.dim() != 2 or x.shape[1] != H * P:
        raise ValueError(f"{fn}: x must be [T, H*P] = [T, {H * P}], got {tuple(x.shape)}")
    t = x.shape[0] if t_rows is None else t_rows
    _shape(dt, (t, H), "dt", fn)
    _shape(B, (t, G * N), "B", fn)
    _shape(C, (t, G * N), "C", fn)
    _shape(z, (t, H * P), "z", fn)
    if D.numel() != H:
        raise ValueError(f"{fn}: D must hold H = {H} values, got {D.numel()}")
    if a_log.numel() not in (H, H * N):
        raise ValueError(f"{fn}: a_log must hold H or H*N values, got {a_log.numel()}")


def _check_cu_seqlens(fn, cu_seqlens):
    """Offsets outside [0, T] are clamped by the kernels; the count must be S+1 >= 2."""
    if cu_seqlens.dim() != 1 or cu_seqlens.numel() < 2:
        raise ValueError(f"{fn}: cu_seqlens must be a 1-D int32 tensor of S+1 >= 2 offsets")


def conv1d_causal(x: torch.Tensor, weight: torch.Tensor, cu_seqlens: torch.Tensor, bias=None,
                  silu: bool = True, out_dtype=None) -> torch.Tensor:
    """Depthwise causal conv + bias + SiLU per sequence (src/mamba2.cpp:1056-1076, 2437-2446).

    x may be a column slice of a wider row-major tensor (unit stride in the last dim).
    """
    if x.stride(1) != 1:
        raise ValueError("conv1d_causal: x must have unit stride in the channel dim")
    _dev(weight, "weight", torch.float32)
    _dev(cu_seqlens, "cu_seqlens", torch.int32)
    _opt(bias, "bias")
    t, c = x.shape
    out_dtype = out_dtype or x.dtype
    out = torch.empty((t, c), dtype=out_dtype, device=x.device)
    call("nsosx_conv1d_causal", _p(x), _dt(x), x.stride(0), _p(weight), _p(bias), _p(cu_seqlens),
         cu_seqlens.numel() - 1, t, c, weight.shape[1], int(silu), _p(out), _DT[out_dtype],
         _stream())
    return out


def _scan_workspace(s, t, H, P, N, chunk_tokens, device):
    nbytes = int(lib().nsosx_scan_fwd_workspace(s, t, H, P, N, chunk_tokens))
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)


def selective_scan_fwd(x, dt, a_log, B, C, D, z, cu_seqlens, H, P, N, G, initial_state=None,
                       want_final: bool = True, chunk_tokens: int | None = -1):
    """Packed ragged faithful scan (src/mamba2.cpp:2602-2675) -> (y [T, H*P], final [S, H*P, N]).

    chunk_tokens: -1 lets the library chunk long sequences in time when the batch cannot
    fill the GPU, 0 never chunks, > 0 forces that chunk length; None calls the unplanned
    entry point (no order pre-pass, no chunking)."""
    _check_scan_shapes("selective_scan_fwd", x, dt, a_log, B, C, D, z, H, P, N, G)
    _check_cu_seqlens("selective_scan_fwd", cu_seqlens)
    t = x.shape[0]
    s = cu_seqlens.numel() - 1
    _shape(initial_state, (s, H * P, N), "initial_state", "selective_scan_fwd")
    if not x.is_cuda:
        raise ValueError("x must be a device tensor")
    if x.stride(1) != 1 or (z is not None and z.stride(1) != 1):
        raise ValueError("selective_scan_fwd: x and z need unit stride in the channel dim")
    for name, v in (("dt", dt), ("B", B), ("C", C)):
        _dev(v, name, x.dtype)
    if z is not None and z.dtype != x.dtype:
        raise ValueError("selective_scan_fwd: z must have x's dtype")
    _dev(a_log, "a_log", torch.float32)
    _dev(D, "D", torch.float32)
    _dev(cu_seqlens, "cu_seqlens", torch.int32)
    _opt(initial_state, "initial_state")
    a_per_state = int(a_log.numel() == H * N and N > 1)
    y = torch.empty((t, H * P), dtype=x.dtype, device=x.device)
    fin = torch.empty((s, H * P, N), dtype=torch.float32, device=x.device) if want_final else None
    if chunk_tokens is None:
        call("nsosx_selective_scan_fwd", _p(x), x.stride(0), _p(dt), _p(a_log), a_per_state,
             _p(B), _p(C), _p(D), _p(z), 0 if z is None else z.stride(0), _p(cu_seqlens), s, t,
             H, P, N, G, _dt(x), _p(initial_state), _p(fin), _p(y), _stream())
    else:
        ws = _scan_workspace(s, t, H, P, N, chunk_tokens, x.device)
        call("nsosx_scan_fwd_planned", _p(x), x.stride(0), None, None, 0, _p(dt), _p(a_log),
             a_per_state, _p(B), _p(C), _p(D), _p(z), 0 if z is None else z.stride(0),
             _p(cu_seqlens), s, t, H, P, N, G, _dt(x), _p(initial_state), _p(fin), _p(y),
             chunk_tokens, _p(ws), _stream())
    return y, fin


def conv_scan_fwd(x_raw, conv_w, conv_b, dt, a_log, B, C, D, z, cu_seqlens, H, P, N, G,
                  initial_state=None, want_final: bool = True, chunk_tokens: int | None = -1):
    """Causal conv + bias + SiLU fused into the scan's staging -> (y, final state).
    chunk_tokens as selective_scan_fwd."""
    _check_scan_shapes("conv_scan_fwd", x_raw, dt, a_log, B, C, D, z, H, P, N, G)
    _check_cu_seqlens("conv_scan_fwd", cu_seqlens)
    t = x_raw.shape[0]
    s = cu_seqlens.numel() - 1
    _shape(initial_state, (s, H * P, N), "initial_state", "conv_scan_fwd")
    if conv_w.dim() != 2 or conv_w.shape[0] != H * P or not 1 <= conv_w.shape[1] <= 8:
        raise ValueError(f"conv_scan_fwd: conv_w must be [H*P, W] = [{H * P}, 1..8], "
                         f"got {tuple(conv_w.shape)}")
    if conv_b is not None and conv_b.numel() != H * P:
        raise ValueError(f"conv_scan_fwd: conv_b must hold H*P = {H * P} values")
    if not x_raw.is_cuda:
        raise ValueError("x_raw must be a device tensor")
    if x_raw.stride(1) != 1 or (z is not None and z.stride(1) != 1):
        raise ValueError("conv_scan_fwd: x and z need unit stride in the channel dim")
    for name, v in (("dt", dt), ("B", B), ("C", C)):
        _dev(v, name, x_raw.dtype)
    _dev(conv_w, "conv_w", torch.float32)
    _opt(conv_b, "conv_b")
    _dev(a_log, "a_log", torch.float32)
    _dev(D, "D", torch.float32)
    _dev(cu_seqlens, "cu_seqlens", torch.int32)
    _opt(initial_state, "initial_state")
    a_per_state = int(a_log.numel() == H * N and N > 1)
    y = torch.empty((t, H * P), dtype=x_raw.dtype, device=x_raw.device)
    fin = (torch.empty((s, H * P, N), dtype=torch.float32, device=x_raw.device)
           if want_final else None)
    if chunk_tokens is None:
        call("nsosx_conv_scan_fwd", _p(x_raw), x_raw.stride(0), _p(conv_w), _p(conv_b),
             conv_w.shape[1], _p(dt), _p(a_log), a_per_state, _p(B), _p(C), _p(D), _p(z),
             0 if z is None else z.stride(0), _p(cu_seqlens), s, t, H, P, N, G, _dt(x_raw),
             _p(initial_state), _p(fin), _p(y), _stream())
    else:
        ws = _scan_workspace(s, t, H, P, N, chunk_tokens, x_raw.device)
        call("nsosx_scan_fwd_planned", _p(x_raw), x_raw.stride(0), _p(conv_w), _p(conv_b),
             conv_w.shape[1], _p(dt), _p(a_log), a_per_state, _p(B), _p(C), _p(D), _p(z),
             0 if z is None else z.stride(0), _p(cu_seqlens), s, t, H, P, N, G, _dt(x_raw),
             _p(initial_state), _p(fin), _p(y), chunk_tokens, _p(ws), _stream())
    return y, fin


def selective_scan_step(x, dt, a_log, B, C, D, z, state, H, P, N, G):
    """Decode step in place on `state` [R, H*P, N] (src/mamba2.cpp:4038-4125) -> y [R, H*P]."""
    _check_scan_shapes("selective_scan_step", x, dt, a_log, B, C, D, z, H, P, N, G)
    r = x.shape[0]
    _shape(state, (r, H * P, N), "state", "selective_scan_step")
    for name, v in (("x", x), ("dt", dt), ("B", B), ("C", C)):
        _dev(v, name, x.dtype)
    if z is not None:
        _dev(z, "z", x.dtype)
    _dev(a_log, "a_log", torch.float32)
    _dev(D, "D", torch.float32)
    _dev(state, "state", torch.float32)
    a_per_state = int(a_log.numel() == H * N and N > 1)
    y = torch.empty_like(x)
    call("nsosx_selective_scan_step", _p(x), _p(dt), _p(a_log), a_per_state, _p(B), _p(C), _p(D),
         _p(z), r, H, P, N, G, _dt(x), _p(state), _p(y), _stream())
    return y


def mamba2_step(x, z, B, C, dt, conv_w, conv_b, ring, a_log, D, norm_w, state, H, P, N, G,
                eps: float = 1e-5, act_bits: int = 8, q=None, act_scale=None, y=None,
                out_proj=None, out=None):
    """The faithful Mamba-2 decode step after its projections, one launch
    (src/mamba2.cpp:4038-4125 through out_proj's input quantization, src/bitlinear.cpp:240-291):
    the conv ring over x | B | C, the state step, RMSNorm(y * SiLU(z)) * norm_w and its int8
    codes, in place on `ring` [R, W-1, H*P + 2*G*N] and `state` [R, H*P, N].

    x, z [R, H*P]; B, C [R, G*N] and dt [R, H] (bias included): column slices of one
    projection output sharing its row stride.  -> (q int8 [R, H*P], act_scale f32 [R],
    y [R, H*P] the pre-gate output).

    out_proj: (packed int32 words [d, H*P / 16], weight_scale, magnitude, bias) of the
    block's ternary out_proj; with it and `out` [R, d] the step also runs the out_proj
    on the codes (nsosx_mamba2_step_out: one launch fewer at one row)."""
    inner, gs = H * P, G * N
    r = x.shape[0]
    _dev(x, "x")
    _dev(z, "z", x.dtype)
    _shape(x, (r, inner), "x", "mamba2_step")
    _shape(z, (r, inner), "z", "mamba2_step")
    stride = B.stride(0) if r > 1 else max(B.stride(0), C.stride(0), dt.stride(0))
    for name, v, n in (("B", B, gs), ("C", C, gs), ("dt", dt, H)):
        if not v.is_cuda or v.dtype != x.dtype or tuple(v.shape) != (r, n) or v.stride(1) != 1:
            raise ValueError(f"mamba2_step: {name} must be a device [{r}, {n}] {x.dtype} view "
                             "with unit column stride")
        if r > 1 and v.stride(0) != stride:
            raise ValueError("mamba2_step: B, C and dt must share one row stride")
    cd = inner + 2 * gs
    _dev(conv_w, "conv_w", torch.float32)
    width = conv_w.shape[1]
    _shape(conv_w, (cd, width), "conv_w", "mamba2_step")
    if conv_b is not None:
        _shape(_dev(conv_b, "conv_b", torch.float32), (cd,), "conv_b", "mamba2_step")
    if width > 1:
        _shape(_dev(ring, "ring", torch.float32), (r, width - 1, cd), "ring", "mamba2_step")
    _shape(_dev(a_log, "a_log", torch.float32), (H,), "a_log", "mamba2_step")
    _shape(_dev(D, "D", torch.float32), (H,), "D", "mamba2_step")
    if norm_w is not None:
        _shape(_dev(norm_w, "norm_w", torch.float32), (inner,), "norm_w", "mamba2_step")
    _shape(_dev(state, "state", torch.float32), (r, inner, N), "state", "mamba2_step")
    if q is None:
        q = torch.empty((r, inner), dtype=torch.int8, device=x.device)
    if act_scale is None:
        act_scale = torch.empty(r, dtype=torch.float32, device=x.device)
    _shape(_dev(q, "q", torch.int8), (r, inner), "q", "mamba2_step")
    _shape(_dev(act_scale, "act_scale", torch.float32), (r,), "act_scale", "mamba2_step")
    if y is None:
        y = torch.empty_like(x)
    _shape(_dev(y, "y", x.dtype), (r, inner), "y", "mamba2_step")
    args = (_p(x), _p(z), _p(B), _p(C), _p(dt), stride, _p(conv_w), _p(conv_b), width,
            _p(ring) if width > 1 else None, _p(a_log), _p(D), _p(norm_w), eps, r, H, P, N, G,
            _dt(x), _p(state), _p(y), _p(q), _p(act_scale), act_bits)
    if out_proj is None:
        call("nsosx_mamba2_step", *args, _stream())
        return q, act_scale, y
    packed, ws, mag, bias = out_proj
    _dev(packed, "out_proj packed")
    d = out.shape[1]
    if packed.numel() != d * inner // 16 or tuple(out.shape) != (r, d) or not out.is_contiguous():
        raise ValueError("mamba2_step: out_proj weights must be [d, H*P/16] words and out [R, d]")
    _opt(mag, "out_proj magnitude")
    _opt(bias, "out_proj bias")
    call("nsosx_mamba2_step_out", *args, _p(packed), ws, d, _p(mag), _p(bias), _p(out), _dt(out),
         _stream())
    return q, act_scale, y


# ---- MoE ------------------------------------------------------------------------

def valid_rows_mask(valid_rows, rows: int, device) -> torch.Tensor | None:
    """The reference's 0/1 valid-row mask on the device (None: every row valid).  A host
    mask is checked as MoERouter::forward checks it (src/jamba.cpp:8145-8153): one entry
    per row, each 0 or 1, else ValueError; a uint8 device tensor is taken as is (the
    routing then treats any nonzero byte as valid, as the reference's device kernel
    does)."""
    if valid_rows is None:
        return None
    if isinstance(valid_rows, torch.Tensor) and valid_rows.is_cuda:
        if valid_rows.dtype != torch.uint8 or valid_rows.numel() != rows:
            raise ValueError("MoERouter valid-row mask size mismatch")
        return valid_rows.contiguous()
    v = np.asarray(valid_rows.cpu() if isinstance(valid_rows, torch.Tensor) else valid_rows)
    if v.size == 0:
        return None
    if v.size != rows:
        raise ValueError("MoERouter valid-row mask size mismatch")
    if np.any((v != 0) & (v != 1)):
        raise ValueError("MoERouter valid-row mask must contain only 0 or 1")
    return torch.from_numpy(v.astype(np.uint8).reshape(-1)).to(device)


def moe_route(logits: torch.Tensor, k: int = 2, select_only: bool = False, valid_rows=None,
              want_loads: bool = False) -> dict:
    """MoERouter::forward(x, valid_rows) from logits + forward_moe's ordered dispatch, on the
    device.  select_only: weights and selected only (one launch), as the sparse decode needs.
    valid_rows: the reference's 0/1 padding mask (host array or uint8 device tensor), None
    for every row valid; padding rows get zero weights, selections -1 and no slots.
    want_loads: also "loads", the per-expert sums of the weights (expert_loads)."""
    _dev(logits, "logits", torch.float32)
    rows, e = logits.shape
    dev = logits.device
    mask = valid_rows_mask(valid_rows, rows, dev)
    out = {
        "weights": torch.empty((rows, e), dtype=torch.float32, device=dev),
        "selected": torch.empty((rows, k), dtype=torch.int32, device=dev),
    }
    if want_loads:
        out["loads"] = torch.empty(e, dtype=torch.float32, device=dev)
    loads = _p(out["loads"]) if want_loads else None
    if select_only:
        call("nsosx_moe_route", _p(logits), _p(mask), rows, e, k, _p(out["weights"]),
             _p(out["selected"]), None, None, None, None, loads, None, _stream())
        return out
    out.update({
        "counts": torch.empty(e, dtype=torch.int32, device=dev),
        "offsets": torch.empty(e + 1, dtype=torch.int32, device=dev),
        "perm": torch.empty(rows * k, dtype=torch.int32, device=dev),
        "slot_of": torch.empty((rows, k), dtype=torch.int32, device=dev),
    })
    ws = torch.empty(max(1, int(lib().nsosx_moe_route_workspace(rows, e))), dtype=torch.int32,
                     device=dev)
    call("nsosx_moe_route", _p(logits), _p(mask), rows, e, k, _p(out["weights"]),
         _p(out["selected"]), _p(out["counts"]), _p(out["offsets"]), _p(out["perm"]),
         _p(out["slot_of"]), loads, _p(ws), _stream())
    return out


def grouped_ternary_gemm(views: LinearViewArray, offsets, perm, q, act_scale, n_out: int,
                         max_rows_per_expert: int, squared_relu: bool = False,
                         gather: bool = True, out_dtype=torch.float32,
                         total_rows: int | None = None) -> torch.Tensor:
    """Per-expert ternary GEMMs over slot segments -> y [slots, n_out] in slot order.

    total_rows: an upper bound on offsets[E] (default: the slot count) so the launch covers
    only the real row tiles; 0 launches max_rows_per_expert rows of tiles per expert."""
    _dev(offsets, "offsets", torch.int32)
    if gather:
        _dev(perm, "perm", torch.int32)
    _dev(q, "q", torch.int8)
    _dev(act_scale, "act_scale", torch.float32)
    slots = int(perm.numel()) if gather else q.shape[0]
    k = q.shape[1]
    y = torch.empty((slots, n_out), dtype=out_dtype, device=q.device)
    total = slots if total_rows is None else int(total_rows)
    call("nsosx_grouped_ternary_gemm", views.ptr, views.count, _p(offsets), _p(perm), int(gather),
         _p(q), _p(act_scale), k, n_out, max_rows_per_expert, total, int(squared_relu), _p(y),
         _DT[out_dtype], _stream())
    return y


def grouped_ternary_gemm_mfma(views: LinearViewArray, offsets, perm, q, act_scale, n_out: int,
                              total_rows: int, squared_relu: bool = False, gather: bool = True,
                              out_dtype=torch.float32, workspace=None) -> torch.Tensor:
    """grouped_ternary_gemm on views holding MFMA-layout weights (compact row tiles).  With a
    workspace (uint8 device tensor of grouped_mfma_workspace_bytes()), the entry that splits a
    sparse last round of tiles along K (nsosx_grouped_ternary_gemm_mfma_ws; same bits)."""
    _dev(offsets, "offsets", torch.int32)
    if gather:
        _dev(perm, "perm", torch.int32)
    _dev(q, "q", torch.int8)
    _dev(act_scale, "act_scale", torch.float32)
    slots = int(perm.numel()) if gather else q.shape[0]
    k = q.shape[1]
    y = torch.empty((slots, n_out), dtype=out_dtype, device=q.device)
    if workspace is None:
        call("nsosx_grouped_ternary_gemm_mfma", views.ptr, views.count, _p(offsets), _p(perm),
             int(gather), _p(q), _p(act_scale), k, n_out, int(total_rows), int(squared_relu),
             _p(y), _DT[out_dtype], _stream())
    else:
        _dev(workspace, "workspace", torch.uint8)
        call("nsosx_grouped_ternary_gemm_mfma_ws", views.ptr, views.count, _p(offsets), _p(perm),
             int(gather), _p(q), _p(act_scale), k, n_out, int(total_rows), int(squared_relu),
             _p(y), _DT[out_dtype], _p(workspace), int(workspace.numel()), _stream())
    return y


def grouped_mfma_workspace_bytes() -> int:
    """Bytes of the split-K tail workspace of nsosx_grouped_ternary_gemm_mfma_ws on the current
    device (2 x CUs x 128 KiB)."""
    n = int(lib().nsosx_grouped_ternary_gemm_mfma_workspace())
    if n <= 0:
        raise NsosxError("nsosx_grouped_ternary_gemm_mfma_workspace", n, "no device")
    return n


def moe_combine(expert_out, slot_of, selected, weights, out_dtype=torch.float32) -> torch.Tensor:
    _dev(slot_of, "slot_of", torch.int32)
    _dev(selected, "selected", torch.int32)
    _dev(weights, "weights", torch.float32)
    rows, e = weights.shape
    k = selected.shape[1]
    dim = expert_out.shape[1]
    out = torch.empty((rows, dim), dtype=out_dtype, device=expert_out.device)
    call("nsosx_moe_combine", _p(expert_out), _dt(expert_out), _p(slot_of), _p(selected),
         _p(weights), rows, e, k, dim, _p(out), _DT[out_dtype], _stream())
    return out


# ---- row norms of the hybrid block and the decode conv ring -----------------

def rmsnorm_gated(y: torch.Tensor, z=None, gamma=None, eps: float = 1e-5,
                  out_dtype=None) -> torch.Tensor:
    """RMSNorm(y * SiLU(z)) * gamma (src/mamba2.cpp:2677-2680); z None: rmsnorm(y) * gamma."""
    _dev(y, "y")
    if y.dim() != 2:
        raise ValueError("rmsnorm_gated: y must be [rows, dim]")
    if z is not None:
        _dev(z, "z", y.dtype)
        if z.shape != y.shape:
            raise ValueError("rmsnorm_gated: z must match y")
    _opt(gamma, "gamma")
    if gamma is not None and gamma.numel() != y.shape[1]:
        raise ValueError("rmsnorm_gated: gamma must have dim elements")
    out = torch.empty(y.shape, dtype=out_dtype or y.dtype, device=y.device)
    call("nsosx_rmsnorm_gated", _p(y), _p(z), _p(gamma), y.shape[0], y.shape[1], eps, _dt(y),
         _p(out), _dt(out), _stream())
    return out


def rmsnorm_gated_quant(y: torch.Tensor, z=None, gamma=None, eps: float = 1e-5, bits: int = 8,
                        want_out: bool = False, out_dtype=None):
    """rmsnorm_gated + the next BitLinear's int8 input quantization (src/mamba2.cpp:2677-2681,
    src/bitlinear.cpp:240-291) -> (q int8 [rows, dim], act_scale f32 [rows], normed or None).
    The normed rows are stored only with want_out (or where the one-pass form does not
    apply: dim % 512 != 0 or dim > 4096)."""
    _dev(y, "y")
    if y.dim() != 2:
        raise ValueError("rmsnorm_gated_quant: y must be [rows, dim]")
    if z is not None:
        _dev(z, "z", y.dtype)
        if z.shape != y.shape:
            raise ValueError("rmsnorm_gated_quant: z must match y")
    _opt(gamma, "gamma")
    rows, dim = y.shape
    if gamma is not None and gamma.numel() != dim:
        raise ValueError("rmsnorm_gated_quant: gamma must have dim elements")
    odt = out_dtype or y.dtype
    one_pass = dim % 512 == 0 and dim <= 4096
    out = torch.empty(y.shape, dtype=odt, device=y.device) if (want_out or not one_pass) else None
    q = torch.empty((rows, dim), dtype=torch.int8, device=y.device)
    s = torch.empty(rows, dtype=torch.float32, device=y.device)
    call("nsosx_rmsnorm_gated_quant", _p(y), _p(z), _p(gamma), rows, dim, eps, _dt(y), _p(out),
         _DT[odt], bits, _p(q), _p(s), _stream())
    return q, s, out


def add_rmsnorm(x: torch.Tensor, delta: torch.Tensor, gamma=None, eps: float = 1e-6,
                want_norm: bool = True):
    """residual = x + delta; norm = rmsnorm(residual) * gamma (src/jamba.cpp:3253, 3286-3290).

    Returns (residual, norm) with norm None when want_norm is False."""
    _dev(x, "x")
    _dev(delta, "delta", x.dtype)
    if x.dim() != 2 or delta.shape != x.shape:
        raise ValueError("add_rmsnorm: x and delta must be the same [rows, dim]")
    _opt(gamma, "gamma")
    res = torch.empty_like(x)
    norm = torch.empty_like(x) if want_norm else None
    call("nsosx_add_rmsnorm", _p(x), _p(delta), _p(gamma), x.shape[0], x.shape[1], eps, _dt(x),
         _p(res), _p(norm), _stream())
    return res, norm


def conv_step(x: torch.Tensor, weight: torch.Tensor, bias, ring, apply_silu: bool = True,
              out_dtype=None) -> torch.Tensor:
    """Decode conv ring step in place on `ring` [R, W-1, C] (src/mamba2.cpp:4072-4090) -> out."""
    if not x.is_cuda or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("conv_step: x must be a device [rows, channels] with unit channel stride")
    _dev(weight, "weight", torch.float32)
    _opt(bias, "bias")
    r, c = x.shape
    w = weight.shape[1]
    if weight.shape[0] != c:
        raise ValueError("conv_step: weight must be [channels, W]")
    if w > 1:
        _dev(ring, "ring", torch.float32)
        if tuple(ring.shape) != (r, w - 1, c):
            raise ValueError("conv_step: ring must be [rows, W-1, channels]")
    out = torch.empty((r, c), dtype=out_dtype or x.dtype, device=x.device)
    call("nsosx_conv_step", _p(x), _dt(x), x.stride(0), r, c, _p(weight), _p(bias), w,
         _p(ring) if w > 1 else None, int(apply_silu), _p(out), _dt(out), _stream())
    return out


# ---- quantization-aware training (fake quant + STE clip) -------------------------

def qat_fake_quant_ternary(w: torch.Tensor, scale: float) -> torch.Tensor:
    """qat_fake_quant_ternary (src/bitnet_gpu_dispatch.cpp:193-217): ternary(w / scale) * scale."""
    _dev(w, "w", torch.float32)
    out = torch.empty_like(w)
    call("nsosx_qat_fake_quant_ternary", _p(w), w.numel(), float(scale), _p(out), _stream())
    return out


def qat_fake_quant_ternary_absmean(w: torch.Tensor):
    """qat_fake_quant_ternary_absmean (src/bitnet_gpu_dispatch.cpp:219-245) -> (out, scale [1])
    with the absmean scale computed and kept on the device."""
    _dev(w, "w", torch.float32)
    out = torch.empty_like(w)
    scale = torch.empty(1, dtype=torch.float32, device=w.device)
    ws = torch.empty(int(lib().nsosx_qat_absmean_workspace(w.numel())), dtype=torch.uint8,
                     device=w.device)
    call("nsosx_qat_fake_quant_ternary_absmean", _p(w), w.numel(), _p(out), _p(scale), _p(ws),
         _stream())
    return out, scale


def qat_fake_quant_activations(x: torch.Tensor, precision_bits: int = 8) -> torch.Tensor:
    """qat_fake_quant_activations (src/bitnet_gpu_dispatch.cpp:247-282): per-row absmax
    quantize-dequantize of the last dimension."""
    _dev(x, "x", torch.float32)
    k = x.shape[-1] if x.dim() else 0
    m = x.numel() // k if k else 0
    out = torch.empty_like(x)
    call("nsosx_qat_fake_quant_activations", _p(x), m, k, int(precision_bits), _p(out), _stream())
    return out


def qat_ste_clip_weight_grad(dW: torch.Tensor, w: torch.Tensor, scale) -> torch.Tensor:
    """qat_ste_clip_weight_grad(_device_scale) (src/bitnet_gpu_dispatch.cpp:284-325), in place
    on dW; `scale` is a float or a device tensor [1]."""
    _dev(dW, "dW", torch.float32)
    _dev(w, "w", torch.float32)
    if dW.shape != w.shape:
        raise ValueError("qat_ste_clip_weight_grad requires identical shapes")
    if isinstance(scale, torch.Tensor):
        _dev(scale, "scale", torch.float32)
        call("nsosx_qat_ste_clip_weight_grad", _p(dW), _p(w), w.numel(), 0.0, _p(scale), _stream())
    else:
        call("nsosx_qat_ste_clip_weight_grad", _p(dW), _p(w), w.numel(), float(scale), None,
             _stream())
    return dW
