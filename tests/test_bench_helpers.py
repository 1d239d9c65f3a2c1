"""CPU checks of bench.py's bookkeeping: the committed rocprofv3 summaries it reads stay
parseable, and the roofline object of the layer carries the fields the bench line reports."""
import importlib.util
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_mod", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_committed_counter_summaries_parse():
    b = _bench()
    traffic = b.pmc_traffic("conv_scan")
    assert isinstance(traffic, int) and traffic > 675_387_136  # at least the algorithmic bytes
    busy = b.pmc_valu_busy("conv + scan")
    assert isinstance(busy, float) and 0.0 < busy <= 100.0
    assert b.pmc_traffic("no_such_stage") is None and b.pmc_valu_busy("no such stage") is None
    # decode kernels: counter bytes at least the algorithmic bytes each extra divides by
    # (128 config-3 weight sets at M = 1; the stacked matrix at M = 16; the config-5 step)
    algo = {"decode_gemv_c3_m1": 539_230_208, "decode_gemv_c3_sweep.m16": 570_458_112,
            "decode_step_c5": 71_319_552}
    for key, lo in algo.items():
        t = b.pmc_traffic(key, b.PMC_DECODE_SUMMARY)
        assert isinstance(t, int) and lo <= t < 1.1 * lo, key


def test_layer_roofline_fields():
    b = _bench()
    T = 40796
    stages = {"in_proj_quant": 0.04, "in_proj_gemm": 0.18, "conv_scan": 0.42,
              "out_proj_quant": 0.075, "out_proj_gemm": 0.08}
    roof, work = b.layer_roofline(T, stages)
    assert roof["kernel"] == "conv_scan" and roof["bound"] == "hbm" and roof["unit"] == "GB/s"
    # algorithmic bytes of the fused conv + scan at config 4: bf16 x, dt, z, y per (token,
    # channel), B and C per token, the fp32 final state per sequence, and the fp32 parameters
    # (A_log per (channel, state); 4 conv taps, conv bias and D per channel)
    assert roof["algorithmic_bytes"] == (T * 2048 * 4 * 2 + T * 16 * 2 * 2 + 32 * 2048 * 16 * 4
                                         + 2048 * 16 * 4 + 2048 * 4 * 6) == 675_387_136
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3
    for key in ("traffic", "valu_issue_bound_ms", "valu_issue_frac", "valu_busy_pct_measured"):
        assert roof[key] is not None
    assert work["in_proj_gemm"][0] == "mfma"
