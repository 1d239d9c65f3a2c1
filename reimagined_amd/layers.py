"""Layer-level compositions over the nsosx operators.

  BitLinear          packed-path BitLinear::forward (src/bitlinear.cpp:439-741)
  HybridMambaLayer   BitLinear in_proj -> causal conv + SiLU -> selective scan
                     gated by SiLU(z) -> BitLinear out_proj over a packed
                     ragged batch (the Mamba layer of JambaBlock::forward,
                     src/jamba.cpp:3158-3375, with Mamba-1 A[D, N])
  MoEFFN             MoERouter::forward from logits + JambaBlock::forward_moe
                     (src/jamba.cpp:3692-3973, 8140-8319): device routing,
                     grouped ternary GEMMs, squared ReLU, weighted combine
  HybridBlock        JambaBlock::forward (src/jamba.cpp:3158-3375) for a Mamba
                     core and an MoE feed-forward: block norms, residual adds

Workspaces are allocated once per shape and reused, so a forward enqueues
kernels only.  Citations are into OXN/nsos/ of vitorGgC569/reimagined.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops
from ._lib import call
from .ops import _DT, _p, _stream


class BitLinear:
    """Packed-path BitLinear: 2-bit ternary weights + per-tensor scale on the device.

    rms_input: the RMS_PERI input norm (eps 1e-6) the reference applies by default.
    """

    def __init__(self, w_float: np.ndarray, device="cuda", bits: int = 8, rms_input: bool = True,
                 magnitude=None, bias=None):
        w_float = np.ascontiguousarray(w_float, dtype=np.float32)
        self.out_features, self.in_features = w_float.shape
        packed, ws = ops.pack_ternary(w_float)
        self.packed = torch.from_numpy(packed.view(np.int32)).to(device)
        self.packed_mfma = self._mfma_layout()
        self.weight_scale = ws
        self.bits = bits
        self.rms_input = rms_input
        self.magnitude = None if magnitude is None else torch.as_tensor(
            magnitude, dtype=torch.float32).to(device)
        self.bias = None if bias is None else torch.as_tensor(bias, dtype=torch.float32).to(device)
        self._ws = {}

    def _mfma_layout(self):
        """The prefill GEMM's copy of the weights (MFMA layout), when K % 128 == 0."""
        return ops.pack_mfma_layout(self.packed) if self.in_features % 128 == 0 else None

    def gemm(self, q, s, m, y, st, magnitude=None, bias=None):
        """The ternary GEMM of m rows of codes into y: on the MFMA-layout words the prefill
        GEMM above 128 rows and the skinny decode kernel at its shapes, else the dispatching
        entry on the reference words (GEMV / small-M MFMA kernels)."""
        if self.packed_mfma is not None and (m > 128 or ops.skinny_shape(m, self.in_features,
                                                                          self.out_features)):
            call("nsosx_ternary_gemm_mfma", _p(q), _p(s), _p(self.packed_mfma),
                 self.weight_scale, m, self.in_features, self.out_features, _p(magnitude),
                 _p(bias), _p(y), _DT[y.dtype], None, st)
        else:
            call("nsosx_ternary_gemm", _p(q), _p(s), _p(self.packed), self.weight_scale, m,
                 self.in_features, self.out_features, _p(magnitude), _p(bias), _p(y),
                 _DT[y.dtype], None, st)

    @classmethod
    def from_packed(cls, packed_u32: np.ndarray, weight_scale: float, out_features: int,
                    in_features: int, device="cuda", **kw):
        """import_packed_state (src/bitlinear.cpp:834-1036): rejects the reserved code 3."""
        self = cls.__new__(cls)
        self.out_features, self.in_features = out_features, in_features
        if in_features % 16 or packed_u32.size != out_features * in_features // 16:
            raise ValueError("packed weights do not match [out, in] with in % 16 == 0")
        self.packed = torch.from_numpy(np.ascontiguousarray(packed_u32).view(np.int32)).to(device)
        bad = ops.find_reserved_code(self.packed, out_features * in_features)
        if bad >= 0:
            raise ValueError(f"packed weights hold the reserved code 3 at index {bad}")
        self.packed_mfma = self._mfma_layout()
        self.weight_scale = float(weight_scale)
        self.bits = kw.get("bits", 8)
        self.rms_input = kw.get("rms_input", True)
        self.magnitude = kw.get("magnitude")
        self.bias = kw.get("bias")
        self._ws = {}
        return self

    def workspace(self, m: int, device):
        ws = self._ws.get(m)
        if ws is None:
            ws = (torch.empty((m, self.in_features), dtype=torch.int8, device=device),
                  torch.empty(m, dtype=torch.float32, device=device),
                  torch.empty(m, dtype=torch.float32, device=device))
            self._ws[m] = ws
        return ws

    def forward_into(self, x: torch.Tensor, y: torch.Tensor, marker=None) -> torch.Tensor:
        """Quantize (with RMS_PERI when set) then the ternary GEMM/GEMV into y.

        marker(name) is called after each kernel (e.g. to record a stream event).
        """
        m = x.shape[0]
        qw, sw, rw = self.workspace(m, x.device)
        st = _stream()
        call("nsosx_quantize_act_i8", _p(x), ops._dt(x), m, self.in_features, self.bits,
             int(self.rms_input), _p(qw), _p(sw), _p(rw), st)
        if marker:
            marker("quant")
        self.gemm(qw, sw, m, y, st, self.magnitude, self.bias)
        if marker:
            marker("gemm")
        return y

    def forward(self, x: torch.Tensor, out_dtype=None) -> torch.Tensor:
        y = torch.empty((x.shape[0], self.out_features), dtype=out_dtype or x.dtype,
                        device=x.device)
        return self.forward_into(x, y)

    def view_entry(self, mfma: bool = False):
        return (self.packed_mfma if mfma else self.packed, self.weight_scale, self.in_features,
                self.out_features, self.magnitude, self.bias)


class HybridMambaLayer:
    """d_model -> in_proj [x | z] -> conv4 + SiLU -> scan -> gate -> out_proj."""

    def __init__(self, params: dict, device="cuda", rms_input: bool = True):
        self.d_model = params["w_in"].shape[1]
        self.d_inner = params["w_out"].shape[1]
        self.d_state = params["a_log"].shape[1]
        self.in_proj = BitLinear(params["w_in"], device, rms_input=rms_input)
        self.out_proj = BitLinear(params["w_out"], device, rms_input=rms_input)
        f32 = dict(dtype=torch.float32, device=device)
        self.conv_w = torch.as_tensor(params["conv_w"], **f32)
        self.conv_b = torch.as_tensor(params["conv_b"], **f32)
        self.a_log = torch.as_tensor(params["a_log"], **f32)
        self.d_skip = torch.as_tensor(params["d_skip"], **f32)
        self._buf = {}

    def _buffers(self, t: int, device, dtype):
        b = self._buf.get(t)
        if b is None:
            b = {
                "xz": torch.empty((t, 2 * self.d_inner), dtype=dtype, device=device),
                "ys": torch.empty((t, self.d_inner), dtype=dtype, device=device),
            }
            self._buf[t] = b
        return b

    def forward(self, x, dt, B, C, cu_seqlens, final_state=None, marker=None, out=None):
        """x [T, d_model]; dt [T, d_inner]; B, C [T, d_state]; cu_seqlens int32 [S+1].

        Returns `out` [T, d_model] (allocated when None; the in_proj and scan buffers stay
        internal).  marker(name), when given, is called after each kernel of the layer.
        """
        t = x.shape[0]
        s = cu_seqlens.numel() - 1
        b = self._buffers(t, x.device, x.dtype)
        di, n = self.d_inner, self.d_state
        mk = (lambda pre: (lambda name: marker(f"{pre}_{name}"))) if marker else (lambda pre: None)
        self.in_proj.forward_into(x, b["xz"], mk("in_proj"))
        xin = b["xz"][:, :di]
        z = b["xz"][:, di:]
        # causal conv + bias + SiLU fused into the scan's input staging; the planned entry
        # orders many sequences once and chunks a batch too small to fill the GPU in time
        ws = b.get(("scan_ws", s))
        if ws is None:
            nbytes = int(ops.lib().nsosx_scan_fwd_workspace(s, t, di, 1, n, -1))
            ws = b[("scan_ws", s)] = torch.empty(max(nbytes, 1), dtype=torch.uint8,
                                                 device=x.device)
        call("nsosx_scan_fwd_planned", _p(xin), xin.stride(0), _p(self.conv_w), _p(self.conv_b),
             self.conv_w.shape[1], _p(dt), _p(self.a_log), 1, _p(B), _p(C), _p(self.d_skip), _p(z),
             z.stride(0), _p(cu_seqlens), s, t, di, 1, n, 1, ops._dt(x), None, _p(final_state),
             _p(b["ys"]), -1, _p(ws), _stream())
        if marker:
            marker("conv_scan")
        if out is None:
            out = torch.empty((t, self.d_model), dtype=x.dtype, device=x.device)
        self.out_proj.forward_into(b["ys"], out, mk("out_proj"))
        return out


class MoEFFN:
    """BASELINE config 5 MoE: top-k routing, expert gate_up -> squared ReLU -> down, combine."""

    def __init__(self, w_up: list, w_down: list, device="cuda", k: int = 2,
                 rms_input: bool = True, hidden_dtype=torch.float32):
        self.experts = len(w_up)
        self.k = k
        self.up = [BitLinear(w, device, rms_input=rms_input) for w in w_up]
        self.down = [BitLinear(w, device, rms_input=rms_input) for w in w_down]
        self.d_model = self.up[0].in_features
        self.d_ff = self.up[0].out_features
        self.rms_input = rms_input
        self.hidden_dtype = hidden_dtype
        self.up_views = ops.LinearViewArray([e.view_entry() for e in self.up], device)
        self.down_views = ops.LinearViewArray([e.view_entry() for e in self.down], device)
        # the prefill GEMMs read the MFMA-layout copies (K % 128 == 0); the sparse decode's
        # GEMVs the reference layout
        self.mfma = all(e.packed_mfma is not None for e in self.up + self.down)
        if self.mfma:
            self.up_views_mfma = ops.LinearViewArray([e.view_entry(True) for e in self.up], device)
            self.down_views_mfma = ops.LinearViewArray([e.view_entry(True) for e in self.down],
                                                       device)
        self._buf = {}

    def _tail_workspace(self, device):
        """The split-K tail workspace of the grouped MFMA GEMMs (one per layer: the up and down
        launches run in stream order)."""
        ws = getattr(self, "_tail_ws", None)
        if ws is None:
            ws = self._tail_ws = torch.empty(ops.grouped_mfma_workspace_bytes(),
                                             dtype=torch.uint8, device=device)
        return ws

    def _buffers(self, rows: int, device):
        b = self._buf.get(rows)
        if b is None:
            slots = rows * self.k
            i32 = dict(dtype=torch.int32, device=device)
            b = {
                "weights": torch.empty((rows, self.experts), dtype=torch.float32, device=device),
                "selected": torch.empty((rows, self.k), **i32),
                "counts": torch.empty(self.experts, **i32),
                "offsets": torch.empty(self.experts + 1, **i32),
                "perm": torch.empty(slots, **i32),
                "slot_of": torch.empty((rows, self.k), **i32),
                "route_ws": torch.empty(max(1, int(ops.lib().nsosx_moe_route_workspace(
                    rows, self.experts))), **i32),
                "q1": torch.empty((rows, self.d_model), dtype=torch.int8, device=device),
                "s1": torch.empty(rows, dtype=torch.float32, device=device),
                "r1": torch.empty(rows, dtype=torch.float32, device=device),
                "h": torch.empty((slots, self.d_ff), dtype=self.hidden_dtype, device=device),
                "q2": torch.empty((slots, self.d_ff), dtype=torch.int8, device=device),
                "s2": torch.empty(slots, dtype=torch.float32, device=device),
                "r2": torch.empty(slots, dtype=torch.float32, device=device),
                "o": torch.empty((slots, self.d_model), dtype=torch.float32, device=device),
            }
            self._buf[rows] = b
        return b

    def forward(self, x: torch.Tensor, logits: torch.Tensor, out_dtype=None,
                marker=None, valid_rows=None) -> dict:
        """Returns {"out": a fresh [rows, d_model] tensor, plus the routing tensors and the
        expert hidden / output rows}.  Those extras are views of this layer's per-row-count
        workspaces: the next forward with the same row count overwrites them.  marker(name),
        when given, is called after each kernel (route, quant_in, up, quant_hidden, down,
        combine).  valid_rows: the reference's 0/1 padding mask (ops.moe_route); padding
        rows take no expert slots and come out as zeros."""
        rows = x.shape[0]
        b = self._buffers(rows, x.device)
        e, k = self.experts, self.k
        st = _stream()
        mk = marker or (lambda name: None)
        mask = ops.valid_rows_mask(valid_rows, rows, x.device)
        call("nsosx_moe_route", _p(logits), _p(mask), rows, e, k, _p(b["weights"]),
             _p(b["selected"]), _p(b["counts"]), _p(b["offsets"]), _p(b["perm"]),
             _p(b["slot_of"]), None, _p(b["route_ws"]), st)
        mk("route")
        call("nsosx_quantize_act_i8", _p(x), ops._dt(x), rows, self.d_model, 8,
             int(self.rms_input), _p(b["q1"]), _p(b["s1"]), _p(b["r1"]), st)
        mk("quant_in")
        slots = rows * k
        if self.mfma:
            tail = self._tail_workspace(x.device)
            call("nsosx_grouped_ternary_gemm_mfma_ws", self.up_views_mfma.ptr, e,
                 _p(b["offsets"]), _p(b["perm"]), 1, _p(b["q1"]), _p(b["s1"]), self.d_model,
                 self.d_ff, slots, 1, _p(b["h"]), _DT[self.hidden_dtype], _p(tail),
                 tail.numel(), st)
        else:
            call("nsosx_grouped_ternary_gemm", self.up_views.ptr, e, _p(b["offsets"]),
                 _p(b["perm"]), 1, _p(b["q1"]), _p(b["s1"]), self.d_model, self.d_ff, rows, slots,
                 1, _p(b["h"]), _DT[self.hidden_dtype], st)
        mk("up")
        call("nsosx_quantize_act_i8", _p(b["h"]), _DT[self.hidden_dtype], slots, self.d_ff, 8,
             int(self.rms_input), _p(b["q2"]), _p(b["s2"]), _p(b["r2"]), st)
        mk("quant_hidden")
        if self.mfma:
            call("nsosx_grouped_ternary_gemm_mfma_ws", self.down_views_mfma.ptr, e,
                 _p(b["offsets"]), None, 0, _p(b["q2"]), _p(b["s2"]), self.d_ff, self.d_model,
                 slots, 0, _p(b["o"]), _DT[torch.float32], _p(tail), tail.numel(), st)
        else:
            call("nsosx_grouped_ternary_gemm", self.down_views.ptr, e, _p(b["offsets"]), None, 0,
                 _p(b["q2"]), _p(b["s2"]), self.d_ff, self.d_model, rows, slots, 0, _p(b["o"]),
                 _DT[torch.float32], st)
        mk("down")
        out = torch.empty((rows, self.d_model), dtype=out_dtype or x.dtype, device=x.device)
        call("nsosx_moe_combine", _p(b["o"]), _DT[torch.float32], _p(b["slot_of"]),
             _p(b["selected"]), _p(b["weights"]), rows, e, k, self.d_model, _p(out),
             _DT[out.dtype], st)
        mk("combine")
        return {"out": out, **{n: b[n] for n in ("weights", "selected", "counts", "offsets",
                                                 "perm", "slot_of", "h", "o")}}

    def decode(self, x: torch.Tensor, logits: torch.Tensor, out_dtype=None,
               valid_rows=None) -> dict:
        """Sparse decode for a few rows (launch_moe_sparse_decode's role): routing on the
        device, then grouped GEMVs over the (row, routed expert) pairs and the combine.
        valid_rows as forward()."""
        rows = x.shape[0]
        b = self._buffers(rows, x.device)
        e, k = self.experts, self.k
        st = _stream()
        mask = ops.valid_rows_mask(valid_rows, rows, x.device)
        call("nsosx_moe_route", _p(logits), _p(mask), rows, e, k, _p(b["weights"]),
             _p(b["selected"]), None, None, None, None, None, None, st)
        nbytes = int(ops.lib().nsosx_moe_sparse_decode_workspace(rows, k, self.d_model,
                                                                 self.d_ff))
        ws = b.get("sparse_ws")
        if ws is None or ws.numel() < nbytes:
            ws = b["sparse_ws"] = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
        out = torch.empty((rows, self.d_model), dtype=out_dtype or x.dtype, device=x.device)
        call("nsosx_moe_sparse_decode", self.up_views.ptr, self.down_views.ptr, e, k,
             _p(b["selected"]), _p(b["weights"]), _p(x), ops._dt(x), rows, self.d_model,
             self.d_ff, int(self.rms_input), _p(ws), _p(out), _DT[out.dtype], st)
        return {"out": out, "weights": b["weights"], "selected": b["selected"], "workspace": ws}


class HybridBlock:
    """JambaBlock::forward with a Mamba core and an MoE feed-forward (src/jamba.cpp:3158-3375):

        h   = rmsnorm(x, 1e-6) * core_gamma        (3175-3179)
        r   = x + mamba(h)                          (3253)
        f   = rmsnorm(r, 1e-6) * ff_gamma           (3286-3290)
        out = r + moe(f)                            (3305-3316)

    gammas None are the non-learnable norms.  The router logits are supplied by the
    caller, or, with `gate_w` [experts, d_model], come from MoERouter's gate projection
    over f (src/jamba.cpp:8140-8319).  The reference marks that gate quantization-
    sensitive unless NSOS_MOE_FP_ROUTER=0 (src/jamba.cpp:8086-8098), so by default it is
    BitLinear's float path: rmsnorm(f, 1e-6) @ gate_w^T * gate_magnitude (+ gate_bias);
    ternary_gate=True builds the ternary BitLinear instead (the NSOS_MOE_FP_ROUTER=0
    behaviour).
    """

    def __init__(self, mamba_params: dict, w_up: list, w_down: list, device="cuda", k: int = 2,
                 core_gamma=None, ff_gamma=None, gate_w=None, core_eps: float = 1e-6,
                 ff_eps: float = 1e-6, gate_magnitude=None, gate_bias=None,
                 ternary_gate: bool = False):
        self.mamba = HybridMambaLayer(mamba_params, device)
        self.moe = MoEFFN(w_up, w_down, device, k=k)
        f32 = dict(dtype=torch.float32, device=device)
        self.core_gamma = None if core_gamma is None else torch.as_tensor(core_gamma, **f32)
        self.ff_gamma = None if ff_gamma is None else torch.as_tensor(ff_gamma, **f32)
        self.gate = None
        self.gate_w = None
        if gate_w is not None and ternary_gate:
            self.gate = BitLinear(gate_w, device, magnitude=gate_magnitude, bias=gate_bias)
        elif gate_w is not None:
            self.gate_w = torch.as_tensor(np.ascontiguousarray(gate_w, np.float32), **f32)
            self.gate_mag = (None if gate_magnitude is None
                             else torch.as_tensor(gate_magnitude, **f32))
            self.gate_bias = None if gate_bias is None else torch.as_tensor(gate_bias, **f32)
        self.core_eps, self.ff_eps = core_eps, ff_eps

    def router_logits(self, f: torch.Tensor) -> torch.Tensor:
        """MoERouter's gate over the normed block input f -> f32 logits [rows, experts]."""
        if self.gate is not None:
            return self.gate.forward(f, out_dtype=torch.float32)
        return ops.linear_f32(f, self.gate_w, rms_input=True, magnitude=self.gate_mag,
                              bias=self.gate_bias)

    def forward(self, x, dt, B, C, cu_seqlens, logits=None, final_state=None,
                valid_rows=None) -> dict:
        """x [T, d_model] (f32 or bf16); the remaining scan inputs as HybridMambaLayer.
        valid_rows: the 0/1 padding mask forward_moe builds from the batch's valid
        lengths (src/jamba.cpp:3708-3710), None for none."""
        ops._dev(cu_seqlens, "cu_seqlens", torch.int32)
        if logits is None and self.gate is None and self.gate_w is None:
            raise ValueError("HybridBlock: pass router logits or build the block with gate_w")
        t, d = x.shape
        h = ops.rmsnorm_gated(x, None, self.core_gamma, eps=self.core_eps)
        core = self.mamba.forward(h, dt, B, C, cu_seqlens, final_state=final_state)
        r, f = ops.add_rmsnorm(x, core, self.ff_gamma, eps=self.ff_eps)
        if logits is None:
            logits = self.router_logits(f)
        ff = self.moe.forward(f, logits, out_dtype=x.dtype, valid_rows=valid_rows)["out"]
        out, _ = ops.add_rmsnorm(r, ff, want_norm=False)
        return {"out": out, "residual": r, "core": core, "ff": ff, "logits": logits,
                "h": h, "f": f}


class Mamba2Block:
    """Faithful Mamba-2 block on the packed path (Mamba2SSD::forward_faithful,
    src/mamba2.cpp:2360-2681; streaming step forward_faithful_step, 3947-4126), with
    the reference's mixed precision (src/mamba2.cpp:584-662):

        x, z   = ternary BitLinear projections of u in exact-linear mode (no input
                 RMSNorm, no magnitude, no bias): one int8 quantization of u shared
                 by the two ternary GEMMs
        B, C   = float linears of u (quantization-sensitive, exact-linear), and
        dt     = a float linear of u plus its bias: one fp32 GEMM over the stacked
                 [w_B; w_C; w_dt] with the bias [0, 0, dt_bias]
        x, B, C = SiLU(causal conv + bias) per sequence (x's conv is fused into
                 the scan's staging; B and C go through the conv kernel)
        y      = faithful scan: per-head A_log [H], P = d_head, G groups, D skip
        out    = out_proj(RMSNorm(y * SiLU(z), eps) * gamma), out_proj a ternary
                 BitLinear in exact-linear mode too (src/mamba2.cpp:514)

    params: w_x [inner, d], w_z [inner, d], w_B [G*N, d], w_C [G*N, d], w_dt [H, d],
    w_out [d, inner], conv_w [inner + 2*G*N, K], conv_b [inner + 2*G*N], a_log [H],
    d_skip [H], norm_w [inner]; optional dt_bias [H] (zeros); shape keys H, P, N, G and
    optional eps (1e-5).  The composition equals the reference's Mamba2SSD::forward on its
    packed deployment path (x, z, out_proj ternary; B, C, dt float) to rounding: the
    oracle's restatement of this chain is pinned against a reference build of Mamba2SSD
    (tests/golden/mamba2_ref.npz).  Activations run in `dtype` (f32 by
    default, the reference's).
    """

    def __init__(self, params: dict, device="cuda", dtype=torch.float32):
        self.H, self.P, self.N, self.G = (int(params[k]) for k in ("H", "P", "N", "G"))
        self.inner = self.H * self.P
        self.gs = self.G * self.N
        self.eps = float(params.get("eps", 1e-5))
        self.dtype = dtype
        self.xz = [BitLinear(params[k], device, rms_input=False) for k in ("w_x", "w_z")]
        self.d_model = self.xz[0].in_features
        f32 = dict(dtype=torch.float32, device=device)
        w_sens = np.concatenate([params["w_B"], params["w_C"], params["w_dt"]]).astype(np.float32)
        self.w_sens = torch.as_tensor(w_sens, **f32)
        dt_bias = params.get("dt_bias")
        bias = np.zeros(2 * self.gs + self.H, np.float32)
        if dt_bias is not None:
            bias[2 * self.gs:] = np.asarray(dt_bias, np.float32)
        self.b_sens = torch.as_tensor(bias, **f32)
        self.out_proj = BitLinear(params["w_out"], device, rms_input=False)
        cw = torch.as_tensor(params["conv_w"], **f32)
        cb = torch.as_tensor(params["conv_b"], **f32)
        self.conv_w_all, self.conv_b_all = cw.contiguous(), cb.contiguous()
        self.K = cw.shape[1]
        i, g = self.inner, self.gs
        self.conv_w = [cw[:i].contiguous(), cw[i:i + g].contiguous(), cw[i + g:].contiguous()]
        self.conv_b = [cb[:i].contiguous(), cb[i:i + g].contiguous(), cb[i + g:].contiguous()]
        self.a_log = torch.as_tensor(params["a_log"], **f32)
        self.d_skip = torch.as_tensor(params["d_skip"], **f32)
        self.norm_w = torch.as_tensor(params["norm_w"], **f32)
        self.views = ops.LinearViewArray([p.view_entry() for p in self.xz], device)
        # one decode row: x, z (packed, 8-bit activations) and B / C / dt (float, with
        # the dt bias) in one grouped launch
        self.decode_views = ops.DecodeViewArray(
            [{"packed": p.packed, "weight_scale": p.weight_scale, "bits": 8,
              "inputs": self.d_model, "outputs": self.inner} for p in self.xz] +
            [{"weight": self.w_sens, "bias": self.b_sens, "inputs": self.d_model,
              "outputs": self.w_sens.shape[0]}], device)

    def _project(self, u: torch.Tensor, contiguous_dt: bool = True) -> list:
        """x, z from one int8 quantization of u (one grouped GEMV launch for <= 8 rows,
        else two ternary GEMMs); B, C, dt from one fp32 GEMM (B and C strided column
        slices; dt contiguous for the prefill scan, a slice too for the decode step)."""
        m = u.shape[0]
        g = self.gs
        if m == 1 and self.d_model % 64 == 0 and self.d_model <= 4096:
            # x / z quantize their row per workgroup; B / C / dt on the float path
            out = ops.grouped_decode_projections(self.decode_views, u[0], out_dtype=self.dtype)
            sens = out[2:3, :self.w_sens.shape[0]]
            dt = sens[:, 2 * g:]
            return [out[0:1, :self.inner], out[1:2, :self.inner], sens[:, :g], sens[:, g:2 * g],
                    dt.contiguous() if contiguous_dt else dt]
        q, s, _ = self.xz[0].workspace(m, u.device)
        st = _stream()
        call("nsosx_quantize_act_i8", _p(u), ops._dt(u), m, self.d_model, 8, 0, _p(q), _p(s),
             None, st)
        if m <= 8:
            y = torch.empty((2, m * self.inner), dtype=self.dtype, device=u.device)
            # both groups read the same codes and scales: zero strides
            call("nsosx_grouped_gemv", self.views.ptr, 2, _p(q), 0, _p(s), 0, m, _p(y),
                 m * self.inner, _DT[self.dtype], st)
            xv, z = y[0].view(m, self.inner), y[1].view(m, self.inner)
        else:
            xv, z = (torch.empty((m, self.inner), dtype=self.dtype, device=u.device)
                     for _ in range(2))
            for p, out in zip(self.xz, (xv, z)):
                p.gemm(q, s, m, out, st)
        sens = ops.linear_f32(u, self.w_sens, bias=self.b_sens, out_dtype=self.dtype)
        dt = sens[:, 2 * g:]
        return [xv, z, sens[:, :g], sens[:, g:2 * g], dt.contiguous() if contiguous_dt else dt]

    def forward(self, u: torch.Tensor, cu_seqlens: torch.Tensor, initial_state=None,
                final_state=None, keep_normed: bool = False, chunk_tokens: int = -1) -> dict:
        """u [T, d_model] over the packed ragged batch cu_seqlens (int32 [S+1]).

        The gated norm and out_proj's input quantization run as one pass
        (nsosx_rmsnorm_gated_quant); the normed rows are stored only with keep_normed.
        chunk_tokens: the scan's time chunking (-1 the library's choice, 0 never, > 0 that
        chunk length)."""
        ops._dev(cu_seqlens, "cu_seqlens", torch.int32)
        xv, z, Bv, Cv, dt = self._project(u)
        Bc = ops.conv1d_causal(Bv, self.conv_w[1], cu_seqlens, self.conv_b[1], True)
        Cc = ops.conv1d_causal(Cv, self.conv_w[2], cu_seqlens, self.conv_b[2], True)
        y, fin = ops.conv_scan_fwd(xv, self.conv_w[0], self.conv_b[0], dt, self.a_log, Bc, Cc,
                                   self.d_skip, None, cu_seqlens, self.H, self.P, self.N, self.G,
                                   initial_state=initial_state, want_final=True,
                                   chunk_tokens=chunk_tokens)
        if final_state is not None:
            final_state.copy_(fin)
        q, s, normed = ops.rmsnorm_gated_quant(y, z, self.norm_w, eps=self.eps,
                                               bits=self.out_proj.bits, want_out=keep_normed)
        out = torch.empty((u.shape[0], self.out_proj.out_features), dtype=self.dtype,
                          device=u.device)
        self.out_proj.gemm(q, s, u.shape[0], out, _stream(), self.out_proj.magnitude,
                           self.out_proj.bias)
        return {"out": out, "x": xv, "z": z, "Bv": Bv, "Cv": Cv, "B": Bc, "C": Cc, "dt": dt,
                "y": y, "normed": normed, "final_state": fin}

    def new_decode_state(self, rows: int, device) -> dict:
        """Zero recurrent state [R, inner, N] and conv ring [R, K-1, inner + 2*G*N]
        (channels x | B | C, the reference's single ring)."""
        f32 = dict(dtype=torch.float32, device=device)
        taps = max(self.K - 1, 1)
        return {"state": torch.zeros((rows, self.inner, self.N), **f32),
                "ring": torch.zeros((rows, taps, self.inner + 2 * self.gs), **f32)}

    def step(self, u: torch.Tensor, dec: dict) -> torch.Tensor:
        """One decode token per row: u [R, d_model]; updates dec's state and ring in place.

        Three launches at one row: the x / z / B / C / dt projections
        (nsosx_grouped_decode_projections), the conv ring + state step, and the out_proj
        GEMV with the gated norm and its quantization as its prologue
        (nsosx_mamba2_step_out).  More rows: the quantization of u and the grouped x / z
        GEMV, the fp32 B / C / dt projection, the step, a norm launch and the out_proj."""
        xv, z, Bv, Cv, dt = self._project(u, contiguous_dt=False)
        m = u.shape[0]
        q, s, _ = self.out_proj.workspace(m, u.device)
        out = torch.empty((m, self.out_proj.out_features), dtype=self.dtype, device=u.device)
        op = self.out_proj
        ops.mamba2_step(xv, z, Bv, Cv, dt, self.conv_w_all, self.conv_b_all,
                        dec["ring"] if self.K > 1 else None, self.a_log, self.d_skip,
                        self.norm_w, dec["state"], self.H, self.P, self.N, self.G, eps=self.eps,
                        act_bits=op.bits, q=q, act_scale=s,
                        out_proj=(op.packed, op.weight_scale, op.magnitude, op.bias), out=out)
        return out

    def capture_step(self, u_static: torch.Tensor, dec: dict):
        """Records one decode step into a HIP graph (torch.cuda.CUDAGraph on ROCm).

        Returns (graph, out): graph.replay() reruns the step on the current contents of
        u_static and dec, writing `out`.  The step launches only kernels (no copies or
        memsets) on the capturing stream, so the graph holds kernel nodes only."""
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step(u_static, {"state": dec["state"].clone(),
                                 "ring": dec["ring"].clone()})  # warm the pools
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = self.step(u_static, dec)
        return g, out
