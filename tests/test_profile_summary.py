"""Host logic of exl3moe.profile_summary on synthetic rocprofv3 CSV files."""
import csv
import json

from exl3moe import profile_summary as ps


def _write(path, rows, fields):
    path.parent.mkdir(parents=True, exist_ok=True)
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def test_traffic_scales_by_copy(tmp_path):
    fields = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    # Counters that see half of the reads and all of the writes.
    _write(tmp_path / "f" / "host" / "1" / "run_counter_collection.csv",
           [{"Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": "FETCH_SIZE", "Counter_Value": 512},
            {"Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": "FETCH_SIZE", "Counter_Value": 3},
            {"Kernel_Name": "void cx::K<1>(x)", "Counter_Name": "FETCH_SIZE", "Counter_Value": 100},
            {"Kernel_Name": "void cx::K<1>(x)", "Counter_Name": "FETCH_SIZE", "Counter_Value": 300},
            {"Kernel_Name": "void cx::K<2>(x)", "Counter_Name": "FETCH_SIZE", "Counter_Value": 7}], fields)
    _write(tmp_path / "w" / "run_counter_collection.csv",
           [{"Kernel_Name": "__amd_rocclr_copyBuffer", "Counter_Name": "WRITE_SIZE", "Counter_Value": 1024},
            {"Kernel_Name": "void cx::K<1>(x)", "Counter_Name": "WRITE_SIZE", "Counter_Value": 10}], fields)
    out = tmp_path / "t.json"
    r = ps.traffic(str(tmp_path / "f"), str(tmp_path / "w"), str(out), 1 << 20, "K<1>", "cmd")
    assert r["copy_calibration"]["fetch_scale"] == 2.0 and r["copy_calibration"]["write_scale"] == 1.0
    assert r["hbm_fetch_bytes_per_launch"] == 200 * 1024 * 2
    assert r["hbm_write_bytes_per_launch"] == 10 * 1024
    assert json.loads(out.read_text())["hbm_bytes_per_launch"] == 200 * 2048 + 10240


def test_stats_table(tmp_path):
    fields = ["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"]
    _write(tmp_path / "s" / "bench_kernel_stats.csv",
           [{"Name": "a", "Calls": 2, "TotalDurationNs": 4000, "AverageNs": 2000, "Percentage": 20, "MinNs": 1000,
             "MaxNs": 3000, "StdDev": 1},
            {"Name": "b", "Calls": 1, "TotalDurationNs": 16000, "AverageNs": 16000, "Percentage": 80,
             "MinNs": 16000, "MaxNs": 16000, "StdDev": 0}], fields)
    out = tmp_path / "s.txt"
    ps.stats(str(tmp_path / "s"), str(out), "the command")
    lines = out.read_text().splitlines()
    assert lines[1] == "# command: the command"
    assert lines[3].split()[-1] == "b" and lines[4].split()[-1] == "a"
    assert lines[4].split()[1] == "2.00"


def test_counters_utilisation(tmp_path):
    fields = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    # One dispatch of 8 XCDs x 1000 cycles: 1024 SIMDs x 1000 SIMD-cycles.
    rows = [{"Kernel_Name": "void cx::G<8>(a)", "Counter_Name": "GRBM_GUI_ACTIVE", "Counter_Value": 8000},
            {"Kernel_Name": "void cx::G<8>(a)", "Counter_Name": "SQ_ACTIVE_INST_VALU", "Counter_Value": 128000},
            {"Kernel_Name": "void cx::G<8>(a)", "Counter_Name": "SQ_VALU_MFMA_BUSY_CYCLES", "Counter_Value": 256000},
            {"Kernel_Name": "void cx::G<8>(a)", "Counter_Name": "SQ_INSTS_MFMA", "Counter_Value": 6000},
            {"Kernel_Name": "void cx::Other(a)", "Counter_Name": "GRBM_GUI_ACTIVE", "Counter_Value": 1}]
    _write(tmp_path / "c" / "run_counter_collection.csv", rows, fields)
    r = ps.counters(str(tmp_path / "c"), str(tmp_path / "c.json"), {"gemm": "G<8>"}, "cmd")
    k = r["kernels"]["gemm"]
    assert k["cycles"] == 1000
    assert k["valu_busy_4cycle_slots"] == 0.5 and k["mfma_busy"] == 0.25
    # 6000 MFMAs x 16384 FLOP in 1000 cycles at 2.4 GHz
    assert abs(k["mfma_issue_TFLOPs"] - 6000 * 16384 / (1000 / 2.4e9) / 1e12) < 0.1
    assert json.loads((tmp_path / "c.json").read_text())["kernels"]["gemm"]["mfma_busy"] == 0.25


def test_counters_wave_cycle_shares(tmp_path):
    # Wave-state counters are divided by SQ_WAVE_CYCLES (same units), per kernel; counters
    # absent from the run are left out, and another kernel's rows are not mixed in.
    fields = ["Kernel_Name", "Counter_Name", "Counter_Value"]
    k = "void cx::G<8>(a)"
    rows = [{"Kernel_Name": k, "Counter_Name": "GRBM_GUI_ACTIVE", "Counter_Value": 8000},
            {"Kernel_Name": k, "Counter_Name": "SQ_WAVE_CYCLES", "Counter_Value": 1000},
            {"Kernel_Name": k, "Counter_Name": "SQ_WAIT_ANY", "Counter_Value": 250},
            {"Kernel_Name": k, "Counter_Name": "SQ_ACTIVE_INST_VALU", "Counter_Value": 400},
            {"Kernel_Name": "void cx::Other(a)", "Counter_Name": "GRBM_GUI_ACTIVE", "Counter_Value": 8000},
            {"Kernel_Name": "void cx::Other(a)", "Counter_Name": "SQ_WAVE_CYCLES", "Counter_Value": 10},
            {"Kernel_Name": "void cx::Other(a)", "Counter_Name": "SQ_WAIT_ANY", "Counter_Value": 10}]
    _write(tmp_path / "w" / "run_counter_collection.csv", rows, fields)
    r = ps.counters(str(tmp_path / "w"), str(tmp_path / "w.json"), {"gemm": "G<8>"}, "cmd")
    sh = r["kernels"]["gemm"]["wave_cycle_shares"]
    assert sh == {"wait_any": 0.25, "active_inst_valu": 0.4}
