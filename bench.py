"""Benchmark of the MI355X hybrid-layer hot path (one GPU).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-extra]

A step is one forward of the hybrid Mamba layer (BitLinear
in_proj 1024 -> 4096, causal conv 4 + SiLU, selective scan d_inner 2048 x
d_state 16 over 32 ragged sequences, gate, BitLinear out_proj 2048 -> 1024;
bf16 activations, fp32 scan state) over one packed batch already resident in
HBM.  `value` is tokens/s of the whole layer.  Per-kernel times come from
stream events recorded between the layer's launches on the launch stream;
the roofline object is for the kernel with the largest share.  The extra
figures are the other two parts of the metric: the prefill ternary GEMM
(config 3) in int8 TOPS and the HBM-bound kernels (decode GEMV over 128
rotated weight sets, the decode step over 8 rotated state buffers) in GB/s.
The CPU baseline times the reference's own BitLinear::forward (oracle/_ref,
built from the reference sources) for the projections and the oracle's
sequential restatement for the conv + scan, on a bounded sample of the same
workload on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _bf16(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).to(dev)


def _f32(torch, a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


class StageTimer:
    """Records a stream event after each kernel; per-stage durations per step."""

    def __init__(self, torch):
        self.torch = torch
        self.events = []

    def start(self):
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record()
        self.events.append(("start", ev))

    def __call__(self, name):
        ev = self.torch.cuda.Event(enable_timing=True)
        ev.record()
        self.events.append((name, ev))

    def totals_ms(self):
        out = {}
        for (_, a), (name, b) in zip(self.events[:-1], self.events[1:]):
            if name == "start":
                continue
            out[name] = out.get(name, 0.0) + a.elapsed_time(b)
        return out


def bench_layer(torch, dev, steps, warmup):
    from reimagined_amd import workloads
    from reimagined_amd.layers import HybridMambaLayer

    params, inp = workloads.config4()
    T = int(inp["cu_seqlens"][-1])
    layer = HybridMambaLayer(params, dev, rms_input=True)
    x = _bf16(torch, inp["x"], dev)
    dt = _bf16(torch, inp["dt"], dev)
    B = _bf16(torch, inp["B"], dev)
    C = _bf16(torch, inp["C"], dev)
    cu = _f32(torch, inp["cu_seqlens"], dev)
    fin = torch.empty((cu.numel() - 1, layer.d_inner, layer.d_state), dtype=torch.float32,
                      device=dev)
    for _ in range(warmup):
        layer.forward(x, dt, B, C, cu, final_state=fin)
    torch.cuda.synchronize()
    # then the same ~150 ms of the layer's own launches every extra gets: `warmup` steps alone
    # (5 under the driver, ~4 ms) leave the clocks still rising when the timed loop starts
    settle_ms = _settle(torch, lambda: layer.forward(x, dt, B, C, cu, final_state=fin))
    _log(f"layer warm: T={T}, settled {settle_ms:.0f} ms")
    # wall-clock timed region: K steps, no per-kernel events
    t0 = time.perf_counter()
    for _ in range(steps):
        layer.forward(x, dt, B, C, cu, final_state=fin)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # per-kernel breakdown: the same K steps with an event after every launch
    timer = StageTimer(torch)
    for _ in range(steps):
        timer.start()
        layer.forward(x, dt, B, C, cu, final_state=fin, marker=timer)
    torch.cuda.synchronize()
    stages = {k: v / steps for k, v in timer.totals_ms().items()}
    return T, wall, stages, params, inp, settle_ms


def bench_mamba2_decode(torch, dev, rows=1, reps=200):
    """Faithful Mamba-2 decode step (d_model 1024, 32 heads x 64, N 16, conv 4), eager vs one
    HIP-graph replay per step.  One row: the x / z / B / C / dt projections in one grouped
    launch, the conv ring + state step, the out_proj GEMV with the gated norm and its
    quantization as its prologue; more rows: five launches.  The step is launch-bound."""
    from reimagined_amd.layers import Mamba2Block
    rng = np.random.default_rng(41)
    d, H, P, N, G, K = 1024, 32, 64, 16, 1, 4
    inner, gs = H * P, G * N
    w = lambda n, k: rng.standard_normal((n, k)).astype(np.float32)
    params = {"w_x": w(inner, d), "w_z": w(inner, d), "w_B": w(gs, d) / 32,
              "w_C": w(gs, d) / 32, "w_dt": w(H, d) / 32, "w_out": w(d, inner),
              "dt_bias": np.full(H, -2.0, np.float32),
              "conv_w": (rng.standard_normal((inner + 2 * gs, K)) * 0.5).astype(np.float32),
              "conv_b": np.zeros(inner + 2 * gs, np.float32),
              "a_log": rng.standard_normal(H).astype(np.float32),
              "d_skip": np.ones(H, np.float32), "norm_w": np.ones(inner, np.float32),
              "H": H, "P": P, "N": N, "G": G}
    blk = Mamba2Block(params, dev)
    dec = blk.new_decode_state(rows, dev)
    u = torch.randn((rows, d), device=dev)
    for _ in range(3):
        blk.step(u, dec)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        blk.step(u, dec)
    torch.cuda.synchronize()
    eager_us = (time.perf_counter() - t0) / reps * 1e6
    g, _ = blk.capture_step(u, dec)
    for _ in range(20):  # replays before the timed ones: the clocks settle
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reps):
        g.replay()
    torch.cuda.synchronize()
    graph_us = (time.perf_counter() - t0) / reps * 1e6
    return {"rows": rows, "eager_us_per_step": round(eager_us, 1),
            "graph_us_per_step": round(graph_us, 1)}


def bench_mamba2_prefill(torch, dev, reps=5, N=16):
    """Faithful Mamba-2 block forward (d_model 1024, 32 heads x 64, d_state N, one A per head,
    conv 4, f32 activations as in the reference) over config 4's 32 ragged sequences
    (T = 40796): the ternary x / z projections, the fp32 B / C / dt projection, B/C conv, fused
    conv + scan, gated norm and out_proj.  N = 64 is the reference model's default
    mamba_d_state (include/nsos_config.h:147); its scan is timed alone as well, with
    stream events around the block's scan launch."""
    from reimagined_amd import workloads
    from reimagined_amd.layers import Mamba2Block
    rng = np.random.default_rng(42)
    d, H, P, G, K = 1024, 32, 64, 1, 4
    inner, gs = H * P, G * N
    w = lambda n, k: rng.standard_normal((n, k)).astype(np.float32)
    params = {"w_x": w(inner, d), "w_z": w(inner, d), "w_B": w(gs, d) / 32,
              "w_C": w(gs, d) / 32, "w_dt": w(H, d) / 32, "w_out": w(d, inner),
              "dt_bias": np.full(H, -2.0, np.float32),
              "conv_w": (rng.standard_normal((inner + 2 * gs, K)) * 0.5).astype(np.float32),
              "conv_b": np.zeros(inner + 2 * gs, np.float32),
              "a_log": rng.standard_normal(H).astype(np.float32),
              "d_skip": np.ones(H, np.float32), "norm_w": np.ones(inner, np.float32),
              "H": H, "P": P, "N": N, "G": G}
    blk = Mamba2Block(params, dev)
    _, inp = workloads.config4()
    cu = torch.from_numpy(inp["cu_seqlens"]).to(dev)
    T = int(inp["cu_seqlens"][-1])
    u = torch.randn((T, d), device=dev)
    _settle(torch, lambda: blk.forward(u, cu))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        blk.forward(u, cu)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    out = {"d_state": N, "tokens": T, "ms": round(ms, 4), "tokens_per_s": round(T / (ms / 1e3), 1)}
    # the scan stage alone, on the block's own projected inputs
    from reimagined_amd import ops
    res = blk.forward(u, cu)
    scan = lambda: ops.conv_scan_fwd(res["x"], blk.conv_w[0], blk.conv_b[0], res["dt"],
                                     blk.a_log, res["B"], res["C"], blk.d_skip, None, cu, H, P, N,
                                     G, want_final=True)
    out["scan_ms"] = round(_time_ms(torch, scan, reps), 4)
    # its roofline: f32 x in and y out per (token, channel), dt per (token, head), B and C
    # per token, the final states; the per-state recurrence bounds it by issue, not HBM
    S = int(cu.numel()) - 1
    scan_bytes = (T * inner * 4 * 2 + T * H * 4 + 2 * T * gs * 4 + S * inner * N * 4
                  + inner * (K + 1) * 4 + 2 * H * 4)
    gbs = scan_bytes / (out["scan_ms"] / 1e3) / 1e9
    out["scan_roofline"] = {"bound": "valu", "bytes": int(scan_bytes), "gbs": round(gbs, 1),
                            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def layer_roofline(T, stages, d_model=1024, d_inner=2048, d_state=16, num_seqs=32):
    """Algorithmic work of each layer kernel per launch (bytes or int8 ops)."""
    work = {
        "in_proj_gemm": ("mfma", 2.0 * T * (2 * d_inner) * d_model),
        "out_proj_gemm": ("mfma", 2.0 * T * d_model * d_inner),
        # bf16 x, dt, z in + y out per (token, channel); B, C per token; fp32 final state
        "scan": ("hbm", T * d_inner * 2 * 4 + T * d_state * 2 * 2 + num_seqs * d_inner * d_state * 4
                 + d_inner * d_state * 4 + d_inner * 4),
        # bf16 x in (strided) + bf16 out per (token, channel)
        "conv_scan": ("hbm", T * d_inner * 2 * 4 + T * d_state * 2 * 2 + num_seqs * d_inner * d_state * 4
                      + d_inner * d_state * 4 + d_inner * 4 * 6),
        "in_proj_quant": ("hbm", T * d_model * (2 + 2 + 1) + T * 8),
        "out_proj_quant": ("hbm", T * d_inner * (2 + 2 + 1) + T * 8),
    }
    name = max((k for k in stages if k in work), key=lambda k: stages[k])
    bound, amount = work[name]
    sec = stages[name] / 1e3
    traffic = pmc_traffic(name)
    if bound == "mfma":
        achieved = amount / sec / 1e12
        roof = {"bound": "mfma", "achieved": round(achieved, 2), "peak": INT8_PEAK_TOPS,
                "unit": "TFLOP/s", "frac": round(achieved / INT8_PEAK_TOPS, 4),
                "traffic": traffic, "kernel": name,
                "note": "int8 ops (TOPS) against the dense int8 MFMA peak"}
    else:
        achieved = amount / sec / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "kernel": name, "algorithmic_bytes": int(amount)}
        if name in ("conv_scan", "scan"):
            # per (token, channel, state) the VALU must issue one exp (two FMA slots), delta * A,
            # the state FMA and the readout FMA; the (delta * x) * B products are formed on the
            # matrix core.  At T*d_inner pairs this issue time exceeds the HBM time
            pairs = T * d_inner
            issue_s = pairs * d_state * (2 + 3) * 4 / 64 / 1024 / 2.4e9
            roof["valu_issue_bound_ms"] = round(issue_s * 1e3, 4)
            roof["valu_issue_frac"] = round(issue_s / sec, 4)
            roof["valu_busy_pct_measured"] = pmc_valu_busy("conv + scan")
            roof["note"] = ("VALU/transcendental-issue bound, not HBM: the recurrence alone needs "
                            f"{issue_s * 1e3:.3f} ms of VALU issue at 2.4 GHz (exp = 2 FMA slots, "
                            "the dx*B products on the matrix core; "
                            f"{issue_s * 6 / 5 * 1e3:.3f} ms with them on the VALU) "
                            f"against {amount / HBM_PEAK_GBS / 1e6:.3f} ms of HBM time; "
                            "valu_issue_frac = that bound / the kernel's time; "
                            "valu_busy_pct_measured = rocprofv3 VALUBusy of the kernel "
                            "(profiles/hybrid_layer_c4_pmc_valu.md)")
    return roof, work


PMC_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                           "hybrid_layer_c4_pmc_traffic.md")
PMC_DECODE_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                  "decode_pmc_traffic.md")


def pmc_traffic(stage: str, summary: str = PMC_SUMMARY):
    """HBM bytes per launch of a stage's kernel, from a committed rocprofv3 PMC summary.

    The summary's table rows read `| stage | kernel | FETCH KiB | WRITE KiB | bytes |`, the
    bytes column already scaled by the copy-kernel calibration stated in that file.  None when
    the summary or the stage's row is absent."""
    try:
        text = open(summary).read()
    except OSError:
        return None
    for line in text.splitlines():
        cells = [c.strip().strip("`") for c in line.strip().strip("|").split("|")]
        if len(cells) == 5 and cells[0] == stage:
            try:
                return int(cells[4].replace(",", ""))
            except ValueError:
                return None
    return None


PMC_VALU_SUMMARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                                "hybrid_layer_c4_pmc_valu.md")


def pmc_valu_busy(stage: str):
    """VALU busy % of a layer stage's kernel from the committed rocprofv3 VALU summary (rows
    `| stage | kernel | dispatches | VALU instructions | active cycles | VALU busy % | wait % |`),
    or None when the summary or the row is absent."""
    try:
        text = open(PMC_VALU_SUMMARY).read()
    except OSError:
        return None
    for line in text.splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) == 7 and cells[0] == stage:
            try:
                return float(cells[5])
            except ValueError:
                return None
    return None


def bench_prefill_gemm(torch, dev, reps=50):
    """Config 3's prefill GEMM (4096 x 2048 x 8192, bf16 out) on the MFMA-layout weights the
    layers use, and on the reference-layout words for comparison; ~150 ms of untimed launches
    first (the first launches after an idle GPU run at lower clocks)."""
    from reimagined_amd import ops, workloads
    from reimagined_amd._lib import call
    from reimagined_amd.ops import _p, _stream
    M, K, N = 4096, 2048, 8192
    c3 = workloads.config3(M=M, K=K, N=N)
    packed, ws = ops.pack_ternary(c3["w"])
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    mf = ops.pack_mfma_layout(pk)
    x = _f32(torch, c3["x"], dev)
    q, s = ops.quantize_activations_bitnet(x, 8)
    y = torch.empty((M, N), dtype=torch.bfloat16, device=dev)

    def run_mfma():
        call("nsosx_ternary_gemm_mfma", _p(q), _p(s), _p(mf), ws, M, K, N, None, None, _p(y), 1,
             None, _stream())

    def run_ref():
        call("nsosx_ternary_gemm_path", _p(q), _p(s), _p(pk), ws, M, K, N, None, None, _p(y), 1,
             None, 1, _stream())
    ms = _time_ms(torch, run_mfma, reps)
    ms_ref = _time_ms(torch, run_ref, reps)
    tops = 2.0 * M * N * K / (ms / 1e3) / 1e12
    return {"shape": [M, K, N], "ms": round(ms, 4), "tops": round(tops, 1),
            "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4), "weights": "mfma layout",
            "reference_layout_ms": round(ms_ref, 4)}


def bench_moe_c5(torch, dev, reps=10):
    """Config 5's MoE FFN prefill: 8192 bf16 tokens, 8 experts (gate_up 1024->4096, squared ReLU,
    down 4096->1024), top-2.  One forward = device routing, RMS + quantize, the grouped up GEMM
    (gathered rows, squared-ReLU epilogue, bf16 hidden), RMS + quantize of the 16384 hidden rows,
    the grouped down GEMM and the combine.  TOPS counts the 2 x 16384 x 2 x 4096 x 1024 int8 ops
    of the two grouped GEMMs over the whole forward's time (a lower bound on the GEMMs' own
    rate)."""
    from reimagined_amd import workloads
    from reimagined_amd.layers import MoEFFN
    moe, _ = workloads.config5(rows=8192, decode_rows=1, d_inner=64)
    layer = MoEFFN(moe["w_up"], moe["w_down"], dev, k=2, rms_input=True,
                   hidden_dtype=torch.bfloat16)
    x = _bf16(torch, moe["x"], dev)
    logits = _f32(torch, moe["logits"], dev)
    _settle(torch, lambda: layer.forward(x, logits))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        layer.forward(x, logits)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    # per kernel: the same forwards with a stream event after every launch
    timer = StageTimer(torch)
    # untimed forwards queued first keep the GPU busy while the host enqueues the instrumented
    # ones, so no stage absorbs host enqueue time (the forward issues ~10 launches from Python)
    for _ in range(20):
        layer.forward(x, logits)
    for _ in range(reps):
        timer.start()
        layer.forward(x, logits, marker=timer)
    torch.cuda.synchronize()
    stages = {n: round(v / reps, 4) for n, v in timer.totals_ms().items()}
    rows, d, f = 8192, 1024, 4096
    gemm_ops = 2.0 * (rows * 2) * f * d  # one grouped GEMM over the 16384 routed slots
    ops_ = 2 * gemm_ops
    tops = ops_ / (ms / 1e3) / 1e12
    per_gemm = {g: {"ms": stages[g], "tops": round(gemm_ops / (stages[g] / 1e3) / 1e12, 1),
                    "frac_int8_peak": round(gemm_ops / (stages[g] / 1e3) / 1e12 / INT8_PEAK_TOPS,
                                            4)}
                for g in ("up", "down")}
    return {"tokens": rows, "experts": 8, "k": 2, "ms": round(ms, 4),
            "tops_whole_forward": round(tops, 1), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
            "tokens_per_s": round(rows / (ms / 1e3), 1), "stages_ms": stages, "gemms": per_gemm}


def bench_decode_gemv(torch, dev, m=1, sets=128, reps=5):
    """Grouped GEMV over `sets` distinct copies of the config-3 weight shape (> MALL)."""
    from reimagined_amd import ops
    K, N = 2048, 8192
    rng = np.random.default_rng(31)
    words = N * K // 16
    # distinct random packed sets generated on the device; a reserved code 3 (both bits
    # set) is turned into code 1 so every word is a valid ternary pattern
    packed = torch.randint(-2**31, 2**31 - 1, (sets, words), dtype=torch.int32, device=dev)
    both = packed & (packed >> 1) & 0x55555555
    packed = (packed ^ (both << 1)).contiguous()
    views = ops.LinearViewArray([(packed[i], 1.0, K, N, None, None) for i in range(sets)], dev)
    q = torch.from_numpy(rng.integers(-127, 128, size=(sets, m, K)).astype(np.int8)).to(dev)
    s = torch.full((sets, m), 0.01, dtype=torch.float32, device=dev)
    y = torch.empty((sets, m, N), dtype=torch.bfloat16, device=dev)
    from reimagined_amd._lib import call
    from reimagined_amd.ops import _p, _stream

    def run():
        call("nsosx_grouped_gemv", views.ptr, sets, _p(q), m * K, _p(s), m, m, _p(y), m * N, 1,
             _stream())
    _settle(torch, run)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        run()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / reps
    bytes_ = sets * (N * K / 4 + m * K + m * N * 2)
    gbs = bytes_ / (ms / 1e3) / 1e9
    return {"m": m, "weight_sets": sets, "bytes_per_launch": int(bytes_), "ms": round(ms, 4),
            "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": pmc_traffic(f"decode_gemv_c3_m{m}", PMC_DECODE_SUMMARY)}


def bench_decode_gemv_sweep(torch, dev, ms=(1, 2, 4, 8, 16, 32), reps=20):
    """Config 3's decode GEMV at M = 1..32 on one tall weight matrix of 128 config-3 weight
    sets stacked in N (N = 128 * 8192, K = 2048; 537 MB, so every launch streams the weights
    from HBM), by the entry BitLinear uses: M = 1 through the dispatching entry on the
    reference words (the VALU GEMV), M >= 2 through nsosx_ternary_gemm_mfma on the MFMA-layout
    copy (the skinny MFMA kernel, shift-and-mask decode)."""
    from reimagined_amd import ops
    from reimagined_amd._lib import call
    from reimagined_amd.ops import _p, _stream
    K, N = 2048, 128 * 8192
    packed = torch.randint(-2**31, 2**31 - 1, (N * K // 16,), dtype=torch.int32, device=dev)
    packed = (packed ^ ((packed & (packed >> 1) & 0x55555555) << 1)).contiguous()
    packed_mfma = ops.pack_mfma_layout(packed)
    rng = np.random.default_rng(32)
    out = {}
    for m in ms:
        q = torch.from_numpy(rng.integers(-127, 128, size=(m, K)).astype(np.int8)).to(dev)
        s = torch.full((m,), 0.01, dtype=torch.float32, device=dev)
        y = torch.empty((m, N), dtype=torch.bfloat16, device=dev)

        def run():
            if m == 1:
                call("nsosx_ternary_gemm", _p(q), _p(s), _p(packed), 1.0, m, K, N, None, None,
                     _p(y), 1, None, _stream())
            else:
                call("nsosx_ternary_gemm_mfma", _p(q), _p(s), _p(packed_mfma), 1.0, m, K, N,
                     None, None, _p(y), 1, None, _stream())
        if m == ms[0]:
            _settle(torch, run)
        for _ in range(10):
            run()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            run()
        b.record()
        torch.cuda.synchronize()
        t = a.elapsed_time(b) / reps
        bytes_ = N * K / 4 + m * K + m * N * 2
        gbs = bytes_ / (t / 1e3) / 1e9
        out[f"m{m}"] = {"ms": round(t, 4), "gbs": round(gbs, 1),
                        "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                        "traffic": pmc_traffic(f"decode_gemv_c3_sweep.m{m}", PMC_DECODE_SUMMARY)}
    del packed, packed_mfma
    return out


def bench_decode_step(torch, dev, reps=8):
    from reimagined_amd import ops, workloads
    _, dec = workloads.config5(rows=16, experts=2, d_model=64, d_ff=64)
    R, Dm, N = dec["state"].shape
    x, dt, z = (_bf16(torch, dec[k], dev) for k in ("x", "dt", "z"))
    B, C = _bf16(torch, dec["B"], dev), _bf16(torch, dec["C"], dev)
    a_log, Dk = _f32(torch, dec["a_log"], dev), _f32(torch, dec["D"], dev)
    states = [_f32(torch, dec["state"], dev) for _ in range(8)]
    for st in states:
        ops.selective_scan_step(x, dt, a_log, B, C, Dk, z, st, Dm, 1, N, 1)
    _settle(torch, lambda: ops.selective_scan_step(x, dt, a_log, B, C, Dk, z, states[0], Dm, 1, N, 1))
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for i in range(reps * len(states)):
        ops.selective_scan_step(x, dt, a_log, B, C, Dk, z, states[i % len(states)], Dm, 1, N, 1)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / (reps * len(states))
    bytes_ = R * Dm * N * 4 * 2 + R * Dm * 2 * 4 + R * N * 2 * 2
    gbs = bytes_ / (ms / 1e3) / 1e9
    return {"rows": R, "ms": round(ms, 4), "gbs": round(gbs, 1),
            "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": int(bytes_),
            "traffic": pmc_traffic("decode_step_c5", PMC_DECODE_SUMMARY)}


def _settle(torch, fn, ms=150.0):
    """Runs fn back to back for about `ms` of wall time: the GPU raises its clocks over
    the first ~100 ms of sustained load, so short HBM-bound timings taken from a cold
    start read low by up to a fifth.  Returns the wall time spent, in ms."""
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(20):
            fn()
        torch.cuda.synchronize()
    return (time.perf_counter() - t0) * 1e3


def _time_ms(torch, fn, reps):
    _settle(torch, fn)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(reps):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / reps


def _time_graph_ms(torch, fn, reps):
    """Device time per call of fn: reps calls captured once into a HIP graph and replayed,
    so host launch overhead (ctypes marshalling, argument checks) stays out of kernels
    that run for only tens of microseconds."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    g.replay()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(3):
        g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / (3 * reps)


def bench_scan_shapes(torch, dev):
    """The scan where the 32-sequence layer batch does not reach: config 2 at batch 1 (one
    512-token sequence over 768 channels, fp32), one 32768-token bf16 prefill over 2048
    channels with the fused conv, 256 ragged sequences of 16-1024 tokens and a
    continuous-batching step of 1024 sequences of 32-64 tokens.  The first two compare the
    time-chunked scan (chunk chosen by the library) with the sequential one; the third the
    once-per-launch longest-first pre-pass with dispatch order; the fourth the planned entry
    with the unplanned one (no ranking in either)."""
    from reimagined_amd import ops, workloads
    out = {}

    def make(T, D, N, lengths, dtype, seed):
        rng = np.random.default_rng(seed)
        p = workloads.scan_params(rng, T, D, N)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dtype).to(dev)
        cu = torch.from_numpy(workloads.cu_seqlens(lengths)).to(dev)
        return p, t, cu

    # config 2: 1 x 512 tokens x 768 channels, fp32, no conv
    p, t, cu = make(512, 768, 16, [512], torch.float32, 2)
    f32 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)
    args = (t(p["x"]), t(p["dt"]), f32(p["a_log"]), t(p["B"]), t(p["C"]), f32(p["D"]),
            t(p["z"]), cu, 768, 1, 16, 1)
    c2 = {}
    for name, ck in (("sequential", 0), ("chunked_auto", -1)):
        c2[f"{name}_ms"] = round(_time_ms(torch, lambda: ops.selective_scan_fwd(
            *args, chunk_tokens=ck), 20), 4)
    bytes_ = 512 * 768 * 4 * 4 + 512 * 16 * 2 * 4 + 768 * 16 * 4 * 2
    c2["bytes"] = bytes_
    c2["chunk_tokens"] = 64
    out["config2_batch1"] = c2

    # one 32768-token prefill, d_inner 2048, N 16, conv 4, bf16
    T, D = 32768, 2048
    rng = np.random.default_rng(7)
    x = torch.randn((T, D), device=dev).to(torch.bfloat16)
    dt = (torch.randn((T, D), device=dev) * 0.5 - 2.0).to(torch.bfloat16)
    z = torch.randn((T, D), device=dev).to(torch.bfloat16)
    B = (torch.randn((T, 16), device=dev) * 0.25).to(torch.bfloat16)
    C = (torch.randn((T, 16), device=dev) * 0.25).to(torch.bfloat16)
    a_log = torch.randn((D, 16), device=dev)
    Dk = torch.randn(D, device=dev)
    cw = torch.randn((D, 4), device=dev) * 0.5
    cb = torch.zeros(D, device=dev)
    cu1 = torch.tensor([0, T], dtype=torch.int32, device=dev)
    long = {}
    for name, ck in (("sequential", 0), ("chunked_auto", -1)):
        long[f"{name}_ms"] = round(_time_ms(torch, lambda: ops.conv_scan_fwd(
            x, cw, cb, dt, a_log, B, C, Dk, z, cu1, D, 1, 16, 1, chunk_tokens=ck), 3), 4)
    bytes_ = T * D * 2 * 4 + T * 16 * 2 * 2 + D * 16 * 4
    long["bytes"] = bytes_
    long["gbs_chunked"] = round(bytes_ / (long["chunked_auto_ms"] / 1e3) / 1e9, 1)
    long["speedup"] = round(long["sequential_ms"] / long["chunked_auto_ms"], 2)
    out["prefill_1x32768"] = long
    del x, dt, z

    # 256 sequences of 16-1024 tokens: the longest-first pre-pass against dispatch order
    lengths = rng.integers(16, 1025, size=256)
    T = int(lengths.sum())
    cus = torch.from_numpy(workloads.cu_seqlens(lengths)).to(dev)
    xs = torch.randn((T, D), device=dev).to(torch.bfloat16)
    dts = (torch.randn((T, D), device=dev) * 0.5 - 2.0).to(torch.bfloat16)
    zs = torch.randn((T, D), device=dev).to(torch.bfloat16)
    Bs = (torch.randn((T, 16), device=dev) * 0.25).to(torch.bfloat16)
    Cs = (torch.randn((T, 16), device=dev) * 0.25).to(torch.bfloat16)
    mid = {"sequences": 256, "tokens": T}
    mid["ordered_prepass_ms"] = round(_time_ms(torch, lambda: ops.conv_scan_fwd(
        xs, cw, cb, dts, a_log, Bs, Cs, Dk, zs, cus, D, 1, 16, 1, chunk_tokens=0), 10), 4)
    mid["unordered_ms"] = round(_time_ms(torch, lambda: ops.conv_scan_fwd(
        xs, cw, cb, dts, a_log, Bs, Cs, Dk, zs, cus, D, 1, 16, 1, chunk_tokens=None), 10), 4)
    out["ragged_256"] = mid
    del xs, dts, zs

    # 1024 sequences of 32-64 tokens (continuous batching), d_inner 2048, conv 4, bf16
    lengths = rng.integers(32, 65, size=1024)
    T = int(lengths.sum())
    cus = torch.from_numpy(workloads.cu_seqlens(lengths)).to(dev)
    xs = torch.randn((T, D), device=dev).to(torch.bfloat16)
    dts = (torch.randn((T, D), device=dev) * 0.5 - 2.0).to(torch.bfloat16)
    zs = torch.randn((T, D), device=dev).to(torch.bfloat16)
    Bs = (torch.randn((T, 16), device=dev) * 0.25).to(torch.bfloat16)
    Cs = (torch.randn((T, 16), device=dev) * 0.25).to(torch.bfloat16)
    many = {"sequences": 1024, "tokens": T}
    # the planned entry (dispatch order above 512 sequences) against the unplanned one
    many["planned_ms"] = round(_time_ms(torch, lambda: ops.conv_scan_fwd(
        xs, cw, cb, dts, a_log, Bs, Cs, Dk, zs, cus, D, 1, 16, 1, chunk_tokens=0), 10), 4)
    many["unplanned_ms"] = round(_time_ms(torch, lambda: ops.conv_scan_fwd(
        xs, cw, cb, dts, a_log, Bs, Cs, Dk, zs, cus, D, 1, 16, 1, chunk_tokens=None), 10), 4)
    many["ordering_share"] = round((many["planned_ms"] - many["unplanned_ms"])
                                   / many["planned_ms"], 4)
    many["tokens_per_s"] = round(T / (many["planned_ms"] / 1e3), 1)
    out["many_short_1024"] = many
    return out


FP32_MFMA_PEAK_TFLOPS = 157.3


def bench_linear_f32(torch, dev):
    """BitLinear's float path (quantization-sensitive layers) on fp32 MFMA: the faithful
    Mamba-2 block's stacked B / C / dt projections over config 4's 40796 tokens (K 1024,
    N 2*16 + 32), and config 5's router gate (RMS_PERI, 8192 x 1024 -> 8).  Device time
    (graph replay): the gate's kernels run for less than the host's launch overhead."""
    from reimagined_amd import ops
    out = {}
    for name, (m, k, n, rms) in {"mamba2_bcdt_c4": (40796, 1024, 64, False),
                                 "router_gate_c5": (8192, 1024, 8, True)}.items():
        x = torch.randn((m, k), device=dev)
        w = torch.randn((n, k), device=dev) / 32
        y = torch.empty((m, n), device=dev)
        fwd = lambda: ops.linear_f32(x, w, rms_input=rms, out=y)
        _settle(torch, fwd)
        ms = _time_graph_ms(torch, fwd, 20)
        tf = 2.0 * m * n * k / (ms / 1e3) / 1e12
        gbs = (m * k * 4 + n * k * 4 + m * n * 4) / (ms / 1e3) / 1e9
        out[name] = {"shape": [m, k, n], "ms": round(ms, 4), "tflops": round(tf, 2),
                     "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
                     "gbs": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    return out


def bench_ste_backward(torch, dev):
    """The packed BitLinear STE backward at an in_proj-sized shape (M 4096 tokens, K 1024,
    N 4096, RMS_PERI, magnitude): dW and d_act are 2*M*N*K fp32 MFMA flops each."""
    from reimagined_amd import ops
    m, k, n = 4096, 1024, 4096
    rng = np.random.default_rng(9)
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    packed, ws = ops.pack_ternary(w)
    wt = torch.from_numpy(w).to(dev)
    pk = torch.from_numpy(packed.view(np.int32)).to(dev)
    x = torch.randn((m, k), device=dev)
    q, s = ops.quantize_activations_bitnet(x, 8, rms_input=True)
    g = torch.randn((m, n), device=dev)
    mag = torch.ones(n, device=dev)
    ms = _time_ms(torch, lambda: ops.bitlinear_ste_backward(x, q, s, wt, pk, ws, g, True, mag,
                                                            True), 5)
    flops = 2 * 2.0 * m * n * k
    tf = flops / (ms / 1e3) / 1e12
    return {"shape": [m, k, n], "ms": round(ms, 4), "tflops": round(tf, 2),
            "frac_fp32_mfma_peak": round(tf / FP32_MFMA_PEAK_TFLOPS, 4)}


def _consumer_wall_us(k: int, n: int):
    """Median host wall time per quantize + GEMV call from the compiled C++ consumer
    (reimagined_amd/host/abi_consumer bench K N: the reference's warmup / 7 x 100-call
    method, benchmarks/bench_decode_gemv.cpp:76-90), or None when it is not built."""
    import subprocess
    from reimagined_amd import build
    if not os.path.exists(build.CONSUMER_OUT):
        return None
    proc = subprocess.run([build.CONSUMER_OUT, "bench", str(k), str(n)], capture_output=True,
                          text=True, timeout=120)
    if proc.returncode != 0:
        _log(f"consumer bench failed: {proc.stderr.strip()}")
        return None
    return json.loads(proc.stdout)["median_wall_us"]


def bench_gemv_published(torch, dev, reps=100):
    """The reference's two published decode-GEMV shapes (M = 1; K x N = 1024 x 4096 and
    4096 x 16384, docs/GPU_MODERNIZATION_RESULTS.md:95-105, bench_decode_gemv.cpp):
      * rotated: grouped over enough distinct weight sets to exceed the 256 MB MALL, so the
        kernel streams HBM (GB/s against peak);
      * resident: back-to-back quantize + GEMV calls on one weight set, as the reference
        measured (its figure is host wall time per call on an RX 7600): the stream time per
        call from events here, and the host wall time per call from the compiled C++
        consumer, the reference's own method."""
    from reimagined_amd import ops
    from reimagined_amd._lib import call
    from reimagined_amd.ops import _p, _stream
    out = {}
    rng = np.random.default_rng(17)
    for k, n in ((1024, 4096), (4096, 16384)):
        words = n * k // 16
        sets = max(2, (512 << 20) // (words * 4))
        packed = torch.randint(-2**31, 2**31 - 1, (sets, words), dtype=torch.int32, device=dev)
        packed = (packed ^ ((packed & (packed >> 1) & 0x55555555) << 1)).contiguous()
        views = ops.LinearViewArray([(packed[i], 1.0, k, n, None, None) for i in range(sets)], dev)
        q = torch.from_numpy(rng.integers(-127, 128, size=(sets, 1, k)).astype(np.int8)).to(dev)
        s = torch.full((sets, 1), 0.01, dtype=torch.float32, device=dev)
        y = torch.empty((sets, 1, n), dtype=torch.float32, device=dev)
        rot = lambda: call("nsosx_grouped_gemv", views.ptr, sets, _p(q), k, _p(s), 1, 1, _p(y), n, 0,
                           _stream())
        ms = _time_ms(torch, rot, 5)
        bytes_ = sets * (n * k / 4 + k + n * 4)
        gbs = bytes_ / (ms / 1e3) / 1e9
        x = torch.randn((1, k), device=dev)
        qw = torch.empty((1, k), dtype=torch.int8, device=dev)
        sw = torch.empty(1, dtype=torch.float32, device=dev)
        y1 = torch.empty((1, n), dtype=torch.float32, device=dev)
        one = packed[0]

        def fwd():
            call("nsosx_bitlinear_forward", _p(x), 0, _p(one), 1.0, 1, k, n, 8, 0, None, None,
                 _p(y1), 0, _p(qw), _p(sw), None, _stream())
        res_ms = _time_ms(torch, fwd, reps)
        out[f"k{k}_n{n}"] = {"rotated_sets": sets, "rotated_us_per_gemv": round(ms / sets * 1e3, 3),
                             "rotated_gbs": round(gbs, 1),
                             "rotated_frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                             "resident_quant_plus_gemv_us": round(res_ms * 1e3, 2)}
        out[f"k{k}_n{n}"]["host_wall_us_cpp"] = _consumer_wall_us(k, n)
        del packed, views
    return out


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(params, inp, min_tokens=3000):
    """The config-4 layer on the host CPU over the first sequences of the same batch (at least
    `min_tokens` tokens).  in_proj and out_proj run the reference's own BitLinear::forward
    (packed path: RMS_PERI with OpenMP, its AVX2 int8 GEMM single-threaded) from oracle/_ref
    when that build is present; the causal conv and the scan, which the reference has no CPU
    Mamba-1 [D, N] path for, run the oracle's sequential restatement (single-threaded)."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import oracle as orc
    from oracle import ref
    import torch
    r = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).float().numpy()
    cu_all = inp["cu_seqlens"]
    S = int(np.searchsorted(cu_all, min_tokens)) if cu_all[-1] > min_tokens else len(cu_all) - 1
    S = max(1, min(S, len(cu_all) - 1))
    T = int(cu_all[S])
    x = r(inp["x"][:T])
    dt = r(inp["dt"][:T])
    B, C = r(inp["B"][:T]), r(inp["C"][:T])
    cu = cu_all[:S + 1].astype(np.int32)
    di = params["w_out"].shape[1]
    n = params["a_log"].shape[1]
    use_ref = ref.available()
    stages = {}
    if use_ref:
        t_in, xz = ref.bitlinear_time_forward(params["w_in"], x, reps=1)
    else:
        pin, wsi, _ = orc.pack_weights(params["w_in"])
        t0 = time.perf_counter()
        xz = orc.bitlinear_forward(x, pin, wsi, 2 * di, rms_input=True)
        t_in = time.perf_counter() - t0
    stages["in_proj"] = {"s": round(t_in, 3), "kind": "reference" if use_ref else "port"}
    t0 = time.perf_counter()
    xc = orc.conv1d_causal(np.ascontiguousarray(xz[:, :di]), params["conv_w"], cu,
                           bias=params["conv_b"], silu_act=True)
    ys, _ = orc.selective_scan(xc, dt, params["a_log"], B, C, params["d_skip"],
                               np.ascontiguousarray(xz[:, di:]), cu, di, 1, n, 1)
    t_scan = time.perf_counter() - t0
    stages["conv_scan"] = {"s": round(t_scan, 3), "kind": "port", "threads": 1}
    if use_ref:
        t_out, _ = ref.bitlinear_time_forward(params["w_out"], ys, reps=1)
    else:
        pout, wso, _ = orc.pack_weights(params["w_out"])
        t0 = time.perf_counter()
        orc.bitlinear_forward(ys, pout, wso, params["w_out"].shape[0], rms_input=True)
        t_out = time.perf_counter() - t0
    stages["out_proj"] = {"s": round(t_out, 3), "kind": "reference" if use_ref else "port"}
    sec = t_in + t_scan + t_out
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = int(omp) if omp and omp.isdigit() else (os.cpu_count() or 1)
    # "reference" only when every stage ran the reference's own code; here the scan is the port
    return {"value": round(T / sec, 2), "unit": "tokens/s", "cores": threads, "kind": "port",
            "cpu_model": cpu_model(), "omp_num_threads": omp,
            "stages": stages,
            "sample": f"the first {S} sequences ({T} tokens) of the config-4 batch through the "
                      f"layer in {sec:.2f} s: in_proj/out_proj by the reference's "
                      f"BitLinear::forward ({'oracle/_ref build' if use_ref else 'oracle port'}; "
                      f"RMSNorm and quantization on {threads} OpenMP threads, the AVX2 int8 "
                      f"GEMM single-threaded), conv + scan by the oracle's sequential "
                      f"restatement on 1 thread (the reference has no CPU Mamba-1 A[D,N] scan)"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # ~20 ms of untimed layer steps: after 3 steps the first 20 timed ones still run ~6 %
    # slower than every later round (the GPU is still raising its clocks)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true")
    ap.add_argument("--only", default=None,
                    help="run only these extras (comma-separated, e.g. prefill_gemm_c3), for "
                         "counter runs")
    ap.add_argument("--skip-layer", action="store_true",
                    help="counter runs: skip the headline layer and print the extras only")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="end with a plain 256 MiB device copy, the known-size kernel that "
                         "FETCH_SIZE / WRITE_SIZE counters are scaled by")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the hot path's kernels run on one MI355X; "
              "multi-GPU sharding is a design note only", file=sys.stderr)
        sys.exit(2)
    import torch
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    import reimagined_amd
    reimagined_amd.lib()
    _log("library loaded")
    extra = {}
    if not args.skip_layer:
        T, wall, stages, params, inp, settle_ms = bench_layer(torch, dev, args.steps, args.warmup)
        ms_step = wall / args.steps * 1e3
        roof, _ = layer_roofline(T, stages)
        _log(f"layer: {ms_step:.3f} ms/step, stages {stages}")
    extras = [
        ("prefill_gemm_c3", "prefill gemm", lambda: bench_prefill_gemm(torch, dev)),
        ("decode_gemv_c3_m1", "decode gemv", lambda: bench_decode_gemv(torch, dev, m=1)),
        ("decode_gemv_c3_sweep", "decode gemv sweep", lambda: bench_decode_gemv_sweep(torch, dev)),
        ("moe_c5", "moe c5", lambda: bench_moe_c5(torch, dev)),
        ("decode_step_c5", "decode step", lambda: bench_decode_step(torch, dev)),
        ("mamba2_prefill", "mamba2 prefill", lambda: bench_mamba2_prefill(torch, dev)),
        ("mamba2_prefill_d_state_64", "mamba2 prefill d_state 64",
         lambda: bench_mamba2_prefill(torch, dev, N=64)),
        ("mamba2_decode_step", "mamba2 decode step", lambda: bench_mamba2_decode(torch, dev)),
        ("scan_shapes", "scan shapes", lambda: bench_scan_shapes(torch, dev)),
        ("linear_f32", "linear f32", lambda: bench_linear_f32(torch, dev)),
        ("ste_backward", "ste backward", lambda: bench_ste_backward(torch, dev)),
        ("gemv_published_shapes", "gemv published shapes", lambda: bench_gemv_published(torch, dev)),
    ]
    only = set(args.only.split(",")) if args.only else None
    if only and only - {k for k, _, _ in extras}:
        print(f"--only: unknown extras {sorted(only - {k for k, _, _ in extras})}",
              file=sys.stderr)
        sys.exit(2)
    if not args.no_extra:
        for key, label, fn in extras:
            if only and key not in only:
                continue
            extra[key] = fn()
            _log(f"{label} {extra[key]}")
    if args.skip_layer:
        print(json.dumps({"extra": extra}), flush=True)
        if args.pmc_calibration:
            _pmc_calibration(torch, dev)
        return
    if not args.no_extra:
        sc = stages.get("conv_scan")
        if sc:
            _, work = layer_roofline(T, {"conv_scan": sc})
            gbs = work["conv_scan"][1] / (sc / 1e3) / 1e9
            extra["scan_c4"] = {"ms": round(sc, 4), "gbs": round(gbs, 1),
                                "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    cpu = None if args.no_cpu else cpu_baseline(params, inp)
    if cpu:
        _log(f"cpu baseline {cpu}")
    line = {
        "metric": "hybrid-layer tokens/s; ternary GEMM int8 TOPS; scan HBM GB/s vs peak",
        "value": round(T * args.steps / wall, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        # untimed layer steps run after the warmup steps, before the timed loop
        "settle_ms": round(settle_ms, 1),
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 GEMM (int32 acc) + fp32 scan, bf16 I/O",
        "data": "synthetic (seeded; ternary weights uniform {-1,0,+1}, random-init)",
        "config": {"workload": "config 4: hybrid Mamba layer d_model 1024, d_inner 2048, "
                               "d_state 16, conv 4, 32 ragged sequences U[64,2048]",
                   "tokens": T, "num_seqs": 32, "rms_peri": True},
        "roofline": roof,
        "cpu_baseline": cpu,
        "stages_ms": {k: round(v, 4) for k, v in stages.items()},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    if args.pmc_calibration:
        _pmc_calibration(torch, dev)


def _pmc_calibration(torch, dev):
    """A plain 256 MiB device copy: the known-size kernel FETCH_SIZE / WRITE_SIZE are
    scaled by."""
    a = torch.empty(256 * 2**20, dtype=torch.uint8, device=dev).fill_(1)
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()


if __name__ == "__main__":
    main()
