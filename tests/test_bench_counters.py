"""bench.py's summary of the MFMA counter pass (CPU: a counter CSV written here)."""
import csv
import importlib.util
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_mod", ROOT / "bench.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def _write(path, dispatches):
    cols = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id", "Thread_Id", "Grid_Size",
            "Kernel_Id", "Kernel_Name", "Workgroup_Size", "LDS_Block_Size", "Scratch_Size", "VGPR_Count",
            "Accum_VGPR_Count", "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp", "End_Timestamp"]
    with open(path, "w", newline="") as fh:
        w = csv.writer(fh)
        w.writerow(cols)
        for i, (name, ns, counters) in enumerate(dispatches, start=1):
            for cname, v in counters.items():
                w.writerow([i, i, "Agent 1", 1, 1, 1, 1, 1, name, 256, 0, 0, 0, 0, 0, cname, v, 1000, 1000 + ns])


def test_counter_summary(bench, tmp_path):
    cus, simds = 256, 1024
    ns = 100_000                       # 100 us per dispatch
    ghz = 2.0
    gui = ghz * ns * bench.N_XCC       # summed over the XCDs
    busy = 0.25 * gui / bench.N_XCC * simds
    ops = 0.25 * simds * bench.INT8_OPS_PER_SIMD_CYCLE * ghz * ns   # a quarter of the peak at 2 GHz
    k256 = "void (anonymous namespace)::gemm_k256<true>((anonymous namespace)::gemm_params)"
    relu = "void (anonymous namespace)::gemm_relu2_q8<127>((anonymous namespace)::gemm_params)"
    warm = {"SQ_VALU_MFMA_BUSY_CYCLES": 1.0, "SQ_INSTS_VALU_MFMA_MOPS_I8": 1.0, "GRBM_GUI_ACTIVE": gui}
    good = {"SQ_VALU_MFMA_BUSY_CYCLES": busy, "SQ_INSTS_VALU_MFMA_MOPS_I8": ops / 512, "GRBM_GUI_ACTIVE": gui}
    rows = [(k256, ns, warm), (relu, ns, warm), ("void other_kernel()", ns, good)]
    rows += [(k256, ns, good), (k256, ns, good), (relu, ns, good), (relu, ns, good)]
    _write(tmp_path / "c.csv", rows)
    res = bench.summarize_counters(tmp_path / "c.csv", cus, skip_first=1)
    for kind, name in (("fp32", "gemm_k256<true>"), ("relu2", "gemm_relu2_q8<127>")):
        r = res[kind]
        assert r["kernels"] == [name]
        assert r["dispatches"] == 2                    # the warm-up third left out
        assert r["mfma_busy_pct"] == pytest.approx(25.0)
        assert r["clock_ghz"] == pytest.approx(ghz)
        assert r["int8_ops_counted_per_launch"] == pytest.approx(ops, rel=1e-9)
        assert r["pct_of_peak_at_clock"] == pytest.approx(25.0)
        assert r["us_per_launch_profiled"] == pytest.approx(100.0)
        assert r["by_kernel"][name]["dispatches"] == 2
        assert r["by_kernel"][name]["int8_tops_profiled"] == r["int8_tops_profiled"]


def test_counter_rates_are_sums(bench, tmp_path):
    """int8_tops_profiled is total ops / total time, not a mean of per-dispatch rates: a
    dispatch twice as long at the same ops weighs in with its time."""
    cus, simds, ghz = 256, 1024, 2.0
    k256 = "void (anonymous namespace)::gemm_k256<false>((anonymous namespace)::gemm_params)"
    rows = []
    for ns in (100_000, 100_000, 100_000, 200_000):      # first is the warm-up quarter
        gui = ghz * ns * bench.N_XCC
        rows.append((k256, ns, {"SQ_VALU_MFMA_BUSY_CYCLES": 0.2 * gui / bench.N_XCC * simds,
                                "SQ_INSTS_VALU_MFMA_MOPS_I8": 1e12 / 512, "GRBM_GUI_ACTIVE": gui}))
    _write(tmp_path / "c.csv", rows)
    r = bench.summarize_counters(tmp_path / "c.csv", cus, skip_first=1)["fp32"]
    assert r["dispatches"] == 3
    assert r["int8_tops_profiled"] == pytest.approx(3e12 / 400_000 / 1e3, rel=1e-3)   # 7500, not 8333
    assert r["mfma_busy_pct"] == pytest.approx(20.0)


def test_short_name(bench):
    assert bench.short_name("void (anonymous namespace)::gemm_k256<true>((anonymous namespace)::gemm_params)") \
        == "gemm_k256<true>"
    assert bench.short_name("void (anonymous namespace)::quantize_kernel<127, 0>(float const*, int, int)") \
        == "quantize_kernel<127, 0>"
    assert bench.short_name("void (anonymous namespace)::gemm_small<2, false, true>((anonymous namespace)::"
                            "gemm_params)") == "gemm_small<2, false, true>"


def test_roofline_of(bench):
    # 10 launches of 1 ms each, 2e12 ops and 1e9 bytes per launch: AI 2000 > ridge -> MFMA bound
    r = bench.roofline_of("k", 10, 10.0, 2e13, 1e10, 5)
    assert r["bound"] == "mfma" and r["achieved"] == pytest.approx(2000.0) and r["frac"] == pytest.approx(0.4)
    assert r["launches_per_step"] == 2 and r["per_launch"]["avg_us"] == pytest.approx(1000.0)
    # no ops (a quantize pass): HBM bound, 1e9 bytes per 1 ms launch = 1000 GB/s
    r = bench.roofline_of("q", 10, 10.0, 0, 1e10, 5)
    assert r["bound"] == "hbm" and r["achieved"] == pytest.approx(1000.0) and r["frac"] == pytest.approx(0.125)


def test_gemm_class(bench):
    assert bench.gemm_class("gemm_small<2, true, true>") == "fp32"
    assert bench.gemm_class("gemm_kernel<false, false, false>") == "fp32"
    assert bench.gemm_class("gemm_relu2_small<63>") == "relu2"
    assert bench.gemm_class("quantize_kernel<127, 0>") is None
