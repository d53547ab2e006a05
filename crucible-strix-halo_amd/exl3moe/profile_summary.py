"""Summaries of rocprofv3 output for the kernels of this library.

    python -m exl3moe.profile_summary stats DIR OUT.txt --cmd "..."
        per-kernel time table from a `rocprofv3 --kernel-trace --stats` run (*kernel_stats.csv)

    python -m exl3moe.profile_summary traffic FETCH_DIR WRITE_DIR OUT.json --copy-bytes N
                                      --kernel SUBSTR --cmd "..."
        HBM bytes per dispatch of the kernels whose name contains SUBSTR, from one
        `--pmc FETCH_SIZE` run and one `--pmc WRITE_SIZE` run of the same program.  Both
        counters are scaled by what they read for a plain device-to-device copy of N bytes
        in the same run (the blit kernel `__amd_rocclr_copyBuffer*`), so the result is in
        bytes whatever the counters' sampling covers.

    python -m exl3moe.profile_summary counters DIR OUT.json --kernel LABEL=SUBSTR ... --cmd "..."
        issue utilisation of the kernels whose name contains SUBSTR from one `--pmc` run with
        GRBM_GUI_ACTIVE, SQ_ACTIVE_INST_VALU, SQ_VALU_MFMA_BUSY_CYCLES and SQ_INSTS_MFMA:
        the fraction of SIMD cycles issuing VALU work and keeping the matrix cores busy,
        and the MFMA issue rate in TFLOP/s against the dense fp16 peak; with SQ_INSTS_LDS
        and SQ_LDS_BANK_CONFLICT (a second pass under the same DIR) the bank-conflict
        cycles per LDS instruction.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import statistics


def _csvs(d: str, suffix: str) -> list[str]:
    return sorted(glob.glob(os.path.join(d, "**", f"*{suffix}"), recursive=True))


def stats(d: str, out: str, cmd: str, top: int = 20) -> None:
    files = _csvs(d, "kernel_stats.csv")
    if not files:
        raise SystemExit(f"no *kernel_stats.csv under {d}")
    rows = []
    for f in files:
        rows += list(csv.DictReader(open(f)))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    with open(out, "w") as o:
        o.write(f"# rocprofv3 kernel statistics\n# command: {cmd}\n")
        o.write(f"# {'calls':>6} {'avg_us':>10} {'min_us':>9} {'max_us':>9} {'total_ms':>9} {'%':>6}  kernel\n")
        for r in rows[:top]:
            o.write(f"  {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:10.2f} {float(r['MinNs']) / 1e3:9.2f} "
                    f"{float(r['MaxNs']) / 1e3:9.2f} {float(r['TotalDurationNs']) / 1e6:9.3f} "
                    f"{100 * float(r['TotalDurationNs']) / total:6.2f}  {r['Name'][:110]}\n")


def _counter(d: str, name: str) -> dict[str, list[float]]:
    """Kernel name -> per-dispatch values of one counter."""
    out: dict[str, list[float]] = {}
    files = _csvs(d, "counter_collection.csv")
    if not files:
        raise SystemExit(f"no *counter_collection.csv under {d}")
    for f in files:
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] == name:
                out.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return out


def traffic(fetch_dir: str, write_dir: str, out: str, copy_bytes: int, kernel: str, cmd: str) -> dict:
    fetch, write = _counter(fetch_dir, "FETCH_SIZE"), _counter(write_dir, "WRITE_SIZE")

    def pick(tab, sub, what):
        vals = [v for k, vs in tab.items() if sub in k for v in vs]
        if not vals:
            raise SystemExit(f"no dispatch of a kernel containing {sub!r} in the {what} run")
        return vals

    # The copy: the largest dispatch of the blit kernel (smaller blits are torch's uploads).
    cf = max(pick(fetch, "copyBuffer", "FETCH_SIZE"))
    cw = max(pick(write, "copyBuffer", "WRITE_SIZE"))
    f_scale = copy_bytes / 1024.0 / cf
    w_scale = copy_bytes / 1024.0 / cw
    kf = pick(fetch, kernel, "FETCH_SIZE")
    kw = pick(write, kernel, "WRITE_SIZE")
    fetch_b = statistics.mean(kf) * 1024 * f_scale
    write_b = statistics.mean(kw) * 1024 * w_scale
    res = {
        "kernel": kernel,
        "command": cmd,
        "dispatches": {"fetch_run": len(kf), "write_run": len(kw)},
        "raw_KiB_per_dispatch": {"FETCH_SIZE": statistics.mean(kf), "WRITE_SIZE": statistics.mean(kw)},
        "copy_calibration": {"bytes": copy_bytes, "FETCH_SIZE_KiB": cf, "WRITE_SIZE_KiB": cw,
                             "fetch_scale": f_scale, "write_scale": w_scale},
        "hbm_fetch_bytes_per_launch": round(fetch_b),
        "hbm_write_bytes_per_launch": round(write_b),
        "hbm_bytes_per_launch": round(fetch_b + write_b),
    }
    with open(out, "w") as o:
        json.dump(res, o, indent=1)
        o.write("\n")
    return res


# MI355X (gfx950): 8 XCDs, 256 CUs x 4 SIMDs, 2.4 GHz peak engine clock, dense fp16 MFMA
# peak 2.5 PFLOP/s; v_mfma_f32_16x16x32_f16 is 2 x 16 x 16 x 32 FLOP.
XCDS, SIMDS, CLOCK_HZ, MFMA_PEAK_TFLOPS, MFMA_FLOP = 8, 1024, 2.4e9, 2500.0, 16384
CUS = SIMDS // 4


def counters(d: str, out: str, kernels: dict[str, str], cmd: str) -> dict:
    """Per-dispatch averages of every counter of the run, and derived issue utilisation.

    GRBM_GUI_ACTIVE is summed over the XCDs (one XCD's count is the kernel's duration in
    cycles); SQ_ACTIVE_INST_VALU counts VALU instructions issued (taken here as 4 cycles
    each, an upper bound); SQ_VALU_MFMA_BUSY_CYCLES counts SIMD cycles with the matrix core
    busy."""
    tabs: dict[str, dict[str, list[float]]] = {}
    for f in _csvs(d, "counter_collection.csv"):
        for r in csv.DictReader(open(f)):
            tabs.setdefault(r["Counter_Name"], {}).setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    if not tabs:
        raise SystemExit(f"no counter rows under {d}")
    res = {"command": cmd, "kernels": {}}
    for label, sub in kernels.items():
        avg = {}
        for name, per in tabs.items():
            vals = [v for k, vs in per.items() if sub in k for v in vs]
            if vals:
                avg[name] = statistics.mean(vals)
        if "GRBM_GUI_ACTIVE" not in avg:
            raise SystemExit(f"no dispatch of a kernel containing {sub!r} with GRBM_GUI_ACTIVE")
        cycles = avg["GRBM_GUI_ACTIVE"] / XCDS
        simd_cycles = cycles * SIMDS
        k = {"substring": sub, "per_dispatch": {n: round(v, 1) for n, v in sorted(avg.items())},
             "cycles": round(cycles), "us_at_peak_clock": round(cycles / CLOCK_HZ * 1e6, 2)}
        if "SQ_ACTIVE_INST_VALU" in avg:
            # Issue slots at 4 cycles each: an upper bound on VALU busy time (simple 32-bit
            # ALU ops and fp32 add/FMA issue in about 2 cycles per wave64 on gfx950).
            k["valu_busy_4cycle_slots"] = round(4 * avg["SQ_ACTIVE_INST_VALU"] / simd_cycles, 4)
        if "SQ_INSTS_VALU" in avg:
            k["valu_instructions_per_simd_cycle"] = round(avg["SQ_INSTS_VALU"] / simd_cycles, 4)
        if "SQ_VALU_MFMA_BUSY_CYCLES" in avg:
            k["mfma_busy"] = round(avg["SQ_VALU_MFMA_BUSY_CYCLES"] / simd_cycles, 4)
        if "SQ_INSTS_MFMA" in avg:
            tf = avg["SQ_INSTS_MFMA"] * MFMA_FLOP / (cycles / CLOCK_HZ) / 1e12
            k["mfma_issue_TFLOPs"] = round(tf, 1)
            k["mfma_issue_frac_of_peak"] = round(tf / MFMA_PEAK_TFLOPS, 4)
        if "SQ_INSTS_LDS" in avg and "SQ_LDS_BANK_CONFLICT" in avg:
            # Bank-conflict stall cycles (summed over the CUs) per LDS instruction issued,
            # and as a share of all CU cycles of the launch.
            k["lds_conflict_cycles_per_lds_instruction"] = round(avg["SQ_LDS_BANK_CONFLICT"] / max(1.0, avg["SQ_INSTS_LDS"]), 4)
            k["lds_conflict_frac_of_cu_cycles"] = round(avg["SQ_LDS_BANK_CONFLICT"] / (cycles * CUS), 4)
        if "SQ_WAVE_CYCLES" in avg:
            # Where the waves' cycles go (each counter summed over waves, as SQ_WAVE_CYCLES):
            # waiting on a waitcnt (memory, LDS, ...), waiting to issue (dependencies, a busy
            # unit), and issuing, per instruction type.
            wc = max(1.0, avg["SQ_WAVE_CYCLES"])
            k["wave_cycle_shares"] = {n[3:].lower(): round(avg[n] / wc, 4) for n in (
                "SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU",
                "SQ_ACTIVE_INST_LDS", "SQ_ACTIVE_INST_VMEM", "SQ_ACTIVE_INST_SCA", "SQ_ACTIVE_INST_MISC") if n in avg}
        res["kernels"][label] = k
    with open(out, "w") as o:
        json.dump(res, o, indent=1)
        o.write("\n")
    return res


def main() -> None:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="what", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("out")
    s.add_argument("--cmd", required=True)
    s.add_argument("--top", type=int, default=20)
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("out")
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--cmd", required=True)
    c = sub.add_parser("counters")
    c.add_argument("dir")
    c.add_argument("out")
    c.add_argument("--kernel", action="append", required=True, help="LABEL=SUBSTR")
    c.add_argument("--cmd", required=True)
    a = ap.parse_args()
    if a.what == "counters":
        ks = dict(x.split("=", 1) for x in a.kernel)
        print(json.dumps(counters(a.dir, a.out, ks, a.cmd)))
    elif a.what == "stats":
        stats(a.dir, a.out, a.cmd, a.top)
    else:
        print(json.dumps(traffic(a.fetch_dir, a.write_dir, a.out, a.copy_bytes, a.kernel, a.cmd)))


if __name__ == "__main__":
    main()
