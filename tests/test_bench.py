"""bench.py's contract pieces that need no GPU: the single-GPU guard and the roofline object."""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "8"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU only" in r.stderr and r.stdout == ""


def test_roofline_divides_the_work_by_the_timed_steps_gpu_time():
    stats = {"median": 0.25, "mean": 0.26, "min": 0.24, "max": 0.31, "launches": 40, "settle_launches": 300,
             "region_ms": 0.2}
    r = bench._roofline("mfma", 2.0e11, stats, bench.PEAK_BF16_TFLOPS, "TFLOP/s", 3.0e8, "k", "algorithmic_flops_per_launch")
    assert abs(r["achieved"] - 1000.0) < 1e-9          # 2e11 flop / 0.2 ms = 1000 TFLOP/s
    assert abs(r["frac"] - 1000.0 / bench.PEAK_BF16_TFLOPS) < 1e-12
    assert r["kernel_ms"] == 0.25 and r["region_ms"] == 0.2 and r["traffic"] == 3.0e8
    assert r["bound"] == "mfma" and r["unit"] == "TFLOP/s" and r["algorithmic_flops_per_launch"] == 2.0e11

    r = bench._roofline("hbm", 4.0e8, stats, bench.PEAK_HBM_GBS, "GB/s", None, "k", "algorithmic_bytes_per_launch")
    assert abs(r["achieved"] - 2000.0) < 1e-9          # 4e8 bytes / 0.2 ms = 2000 GB/s
    assert abs(r["frac"] - 0.25) < 1e-12 and r["traffic"] is None


def test_trace_summary_keeps_only_the_timed_launches(tmp_path):
    # A kernel trace with settle / warm-up launches before the timed ROCTx range and evented ones
    # after it: only the two launches inside the range count.
    kt = tmp_path / "run_kernel_trace.csv"
    kt.write_text("Kind,Kernel_Name,Start_Timestamp,End_Timestamp\n"
                  "KERNEL_DISPATCH,k,1000,400000\n"            # warm-up: 399 us
                  "KERNEL_DISPATCH,k,500000,780000\n"          # timed: 280 us
                  "KERNEL_DISPATCH,k,781000,1051000\n"         # timed: 270 us
                  "KERNEL_DISPATCH,k,2000000,2300000\n")       # after the range
    mk = tmp_path / "run_marker_api_trace.csv"
    mk.write_text("Domain,Function,Start_Timestamp,End_Timestamp\n"
                  "MARKER_CORE_API,bench:prefill:2:2.75e+11:TFLOP/s,450000,1100000\n")
    (rec,) = bench.trace_summary(str(tmp_path))
    assert rec["workload"] == "prefill" and rec["steps"] == 2
    assert rec["kernels"]["k"]["calls"] == 2
    assert abs(rec["kernels"]["k"]["mean_us"] - 275.0) < 1e-9
    assert abs(rec["kernel_ms_per_step"] - 0.275) < 1e-12
    assert abs(rec["achieved"] - 1000.0) < 1e-6       # 2.75e11 flop / 0.275 ms
