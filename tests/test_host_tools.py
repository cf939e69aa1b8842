"""CPU tests of the measurement tooling: the rocprofv3 summaries behind profiles/ and bench.py's
roofline fields, the byte / FLOP conventions of workloads.py, and bench.py's one-GPU contract."""
from __future__ import annotations

import csv
import pathlib
import subprocess
import sys

import pytest

from hyperkernels_amd import rocprof_summary as rs
from hyperkernels_amd import workloads as W

ROOT = pathlib.Path(__file__).resolve().parents[1]

COUNTER_FIELDS = ["Correlation_Id", "Dispatch_Id", "Agent_Id", "Queue_Id", "Process_Id",
                  "Thread_Id", "Grid_Size", "Kernel_Id", "Kernel_Name", "Workgroup_Size",
                  "LDS_Block_Size", "Scratch_Size", "VGPR_Count", "Accum_VGPR_Count",
                  "SGPR_Count", "Counter_Name", "Counter_Value", "Start_Timestamp",
                  "End_Timestamp"]


def _counters(d: pathlib.Path, rows):
    """Writes a rocprofv3-style counter_collection.csv; rows = (dispatch, kernel, counter,
    value, start_ns, end_ns). A counter may appear several times per dispatch (per XCD)."""
    d.mkdir(parents=True, exist_ok=True)
    with open(d / "1_counter_collection.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=COUNTER_FIELDS)
        w.writeheader()
        for i, (disp, kern, name, val, t0, t1) in enumerate(rows):
            w.writerow({"Correlation_Id": i, "Dispatch_Id": disp, "Agent_Id": 1, "Queue_Id": 1,
                        "Process_Id": 7, "Thread_Id": 7, "Grid_Size": 256, "Kernel_Id": 1,
                        "Kernel_Name": kern, "Workgroup_Size": 256, "LDS_Block_Size": 0,
                        "Scratch_Size": 0, "VGPR_Count": 8, "Accum_VGPR_Count": 0,
                        "SGPR_Count": 16, "Counter_Name": name, "Counter_Value": val,
                        "Start_Timestamp": t0, "End_Timestamp": t1})
    with open(d / "1_agent_info.csv", "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Agent_Type", "Num_Xcc", "Simd_Count"])
        w.writeheader()
        w.writerow({"Agent_Type": "CPU", "Num_Xcc": 1, "Simd_Count": 0})
        w.writerow({"Agent_Type": "GPU", "Num_Xcc": 8, "Simd_Count": 1024})


def test_traffic_calibrates_each_counter_on_the_copy(tmp_path):
    copy = "void at::native::vectorized_elementwise_kernel<4, MulFunctor<float>>(int)"
    adam = "(anonymous namespace)::adam_plan_kernel(TensorEntry const*)"
    gib = 1 << 30
    # the copy moves 1 GiB each way; FETCH_SIZE reads half of it (KiB), WRITE_SIZE all of it
    _counters(tmp_path / "cf", [(1, copy, "FETCH_SIZE", gib / 2 / 1024, 0, 1)])
    _counters(tmp_path / "cw", [(1, copy, "WRITE_SIZE", gib / 1024, 0, 1)])
    # two AdamW dispatches: 1000 KiB and 1200 KiB of FETCH_SIZE (mean 1100), split over 2 XCDs
    _counters(tmp_path / "sf", [(5, adam, "FETCH_SIZE", 600.0, 0, 1),
                                (5, adam, "FETCH_SIZE", 400.0, 0, 1),
                                (9, adam, "FETCH_SIZE", 1200.0, 0, 1)])
    _counters(tmp_path / "sw", [(5, adam, "WRITE_SIZE", 300.0, 0, 1),
                                (9, adam, "WRITE_SIZE", 300.0, 0, 1)])
    lines = rs.traffic(tmp_path / "sf", tmp_path / "sw", tmp_path / "cf", tmp_path / "cw", gib)
    assert "scale 2.0000" in lines[0] and "scale 1.0000" in lines[0]
    (adam_line,) = [ln for ln in lines if ln.startswith("traffic: adamw_148 ")]
    kv = dict(x.split("=") for x in adam_line.split()[2:])
    assert float(kv["fetch_bytes"]) == pytest.approx(1100 * 1024 * 2.0)
    assert float(kv["write_bytes"]) == pytest.approx(300 * 1024)
    assert float(kv["traffic_bytes"]) == pytest.approx(1100 * 2048 + 300 * 1024)
    # bench.py reads the committed summary back through read_traffic
    summary = tmp_path / "traffic.txt"
    summary.write_text("# header\n" + "\n".join(lines) + "\n")
    assert rs.read_traffic(summary)["adamw_148"] == pytest.approx(1100 * 2048 + 300 * 1024)
    assert rs.read_traffic(tmp_path / "missing.txt") == {}


def test_pmc_derives_clock_mfma_busy_and_lds_conflicts(tmp_path):
    kern = "void (anonymous namespace)::bgemm_tiled<true, false, false>(int, int)"
    # one dispatch of 100 us; GRBM_GUI_ACTIVE summed over 8 XCDs = 8 * 200,000 cycles (2 GHz);
    # the matrix core busy for half of 1024 SIMDs x 200,000 cycles; a quarter of LDS cycles
    # are bank conflicts. Counters come from two runs (one counter set each).
    _counters(tmp_path / "r1", [(3, kern, "GRBM_GUI_ACTIVE", 8 * 200_000, 0, 100_000),
                                (3, kern, "SQ_VALU_MFMA_BUSY_CYCLES", 1024 * 100_000, 0, 100_000)])
    _counters(tmp_path / "r2", [(4, kern, "GRBM_GUI_ACTIVE", 8 * 200_000, 0, 100_000),
                                (4, kern, "SQ_LDS_IDX_ACTIVE", 4000, 0, 100_000),
                                (4, kern, "SQ_LDS_BANK_CONFLICT", 1000, 0, 100_000)])
    out = rs.pmc("bgemm_tiled", [tmp_path / "r1", tmp_path / "r2"])
    derived = {ln.split()[0]: float(ln.split()[1]) for ln in out if ln.startswith("  ")
               and ln.split()[0] in ("clock_ghz", "mfma_busy", "lds_conflict")}
    assert derived["clock_ghz"] == pytest.approx(2.0)
    assert derived["mfma_busy"] == pytest.approx(0.5)
    assert derived["lds_conflict"] == pytest.approx(0.25)
    assert out[0].startswith("kernel bgemm_tiled<true, false, false>: dispatches/run 1")
    assert rs.pmc("no_such_kernel", [tmp_path / "r1"]) == []


def test_workload_conventions():
    # reference README byte conventions and the 4 B T^2 d / 2.5x attention FLOP counts
    assert W.GPT2_NUM_PARAMS == sum(W.numel(s) for s in W.gpt2_param_shapes()) == 124_439_808
    assert len(W.gpt2_param_shapes()) == 148
    assert W.adamw_bytes(10) == 280
    assert W.gelu_fwd_bytes(10, 2) == 40 and W.gelu_bwd_bytes(10, 2) == 60
    assert W.ce_fwd_bytes(2, 5) == 40 and W.ce_bwd_bytes(2, 5) == 80
    assert W.ln_fwd_bytes(2, 3) == 48 and W.ln_bwd_bytes(2, 3, 2) == 36
    assert W.attn_fwd_flop(1, 1, 4, 2, False) == 4 * 4 * 4 * 2
    assert W.attn_fwd_flop(1, 1, 4, 2, True) == W.attn_fwd_flop(1, 1, 4, 2, False) // 2
    assert W.attn_bwd_flop(8, 12, 1024, 64, False) == 5 * W.attn_fwd_flop(8, 12, 1024, 64,
                                                                          False) // 2
    assert W.gemm_flop(2, 3, 4, batch=5) == 240
    assert W.PEAK_TFLOPS["bf16x3"] == pytest.approx(W.PEAK_TFLOPS["bf16"] / 3)


def test_bench_refuses_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=120)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr
