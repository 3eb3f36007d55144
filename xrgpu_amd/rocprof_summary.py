"""Summarise rocprofv3 output for one kernel into a short text record.

Inputs are rocprofv3 CSV files (``--output-format csv``):

* ``--stats``: ``*_kernel_stats.csv`` of a ``--kernel-trace --stats`` run;
* ``--fetch`` / ``--write``: ``*_counter_collection.csv`` of a ``--pmc
  FETCH_SIZE`` and a ``--pmc WRITE_SIZE`` run of the same command;
* ``--cal-fetch`` / ``--cal-write``: the same counters for a plain device copy
  of ``--cal-bytes`` bytes (read once, written once), which scale the raw
  counters to bytes: factor = cal_bytes / (counter KiB * 1024).

The record gives the average kernel duration, the calibrated HBM bytes per
launch (``traffic``) and their ratio to the algorithmic bytes. ``bench.py``
reads the ``traffic_bytes_per_launch`` line.

Usage::

    python -m xrgpu_amd.rocprof_summary --kernel k_gemv_q4 --dispatch-name gemv_q4_mfma \\
        --algorithmic-bytes 33067008 --stats S.csv --fetch F.csv --write W.csv \\
        --cal-fetch CF.csv --cal-write CW.csv --cal-kernel copyBuffer --cal-bytes 268435456 \\
        --command "..." --out profiles/decode_up_m1_gemv.md
"""
from __future__ import annotations

import argparse
import csv
import statistics


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def kernel_stats(path, kernel):
    for r in _rows(path):
        if kernel in r["Name"]:
            return {"name": r["Name"], "calls": int(r["Calls"]), "avg_ns": float(r["AverageNs"]),
                    "min_ns": float(r["MinNs"]), "max_ns": float(r["MaxNs"])}
    raise KeyError(f"{kernel} not in {path}")


def counter_avg(path, kernel, counter):
    vals = [float(r["Counter_Value"]) for r in _rows(path)
            if kernel in r["Kernel_Name"] and r["Counter_Name"] == counter]
    if not vals:
        raise KeyError(f"{counter} for {kernel} not in {path}")
    return statistics.fmean(vals), len(vals)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--kernel", required=True, help="substring of the kernel symbol")
    ap.add_argument("--dispatch-name", required=True, help="name the dispatcher reports for this kernel")
    ap.add_argument("--workload", required=True)
    ap.add_argument("--algorithmic-bytes", type=int, required=True)
    ap.add_argument("--stats", required=True)
    ap.add_argument("--fetch")
    ap.add_argument("--write")
    ap.add_argument("--cal-fetch")
    ap.add_argument("--cal-write")
    ap.add_argument("--cal-kernel", default="copyBuffer")
    ap.add_argument("--cal-bytes", type=int, default=268435456)
    ap.add_argument("--pmc", action="append", default=[],
                    help="*_counter_collection.csv of a further --pmc run (repeatable): every counter recorded "
                         "for the kernel is listed as its per-dispatch mean")
    ap.add_argument("--cus", type=int, default=256, help="compute units, for the MFMA busy fraction")
    ap.add_argument("--xcds", type=int, default=8,
                    help="GRBM_GUI_ACTIVE instances summed by rocprofv3 (one per XCD on MI355X)")
    ap.add_argument("--command", required=True, help="the command line that produced the CSVs")
    ap.add_argument("--out", required=True)
    a = ap.parse_args(argv)

    st = kernel_stats(a.stats, a.kernel)
    lines = [f"# rocprofv3 summary: {a.workload}", "",
             f"kernel: {st['name']}", f"dispatch_name: {a.dispatch_name}",
             f"calls: {st['calls']}", f"avg_duration_ns: {st['avg_ns']:.1f}",
             f"min_duration_ns: {st['min_ns']:.1f}", f"max_duration_ns: {st['max_ns']:.1f}",
             f"algorithmic_bytes_per_launch: {a.algorithmic_bytes}",
             f"algorithmic_GBps_at_avg: {a.algorithmic_bytes / st['avg_ns']:.1f}"]
    if a.fetch and a.write and a.cal_fetch and a.cal_write:
        fk, nf = counter_avg(a.fetch, a.kernel, "FETCH_SIZE")
        wk, nw = counter_avg(a.write, a.kernel, "WRITE_SIZE")
        cf, _ = counter_avg(a.cal_fetch, a.cal_kernel, "FETCH_SIZE")
        cw, _ = counter_avg(a.cal_write, a.cal_kernel, "WRITE_SIZE")
        ff = a.cal_bytes / (cf * 1024.0)
        fw = a.cal_bytes / (cw * 1024.0)
        traffic = fk * 1024.0 * ff + wk * 1024.0 * fw
        lines += ["", f"FETCH_SIZE_KiB_per_dispatch: {fk:.1f} (n={nf})", f"WRITE_SIZE_KiB_per_dispatch: {wk:.1f} (n={nw})",
                  f"copy_calibration: {a.cal_bytes} B copy reads FETCH_SIZE {cf:.1f} KiB, WRITE_SIZE {cw:.1f} KiB",
                  f"fetch_factor: {ff:.4f}", f"write_factor: {fw:.4f}",
                  f"traffic_bytes_per_launch: {traffic:.0f}",
                  f"traffic_over_algorithmic: {traffic / a.algorithmic_bytes:.4f}"]
    if a.pmc:
        vals = {}
        for path in a.pmc:
            for r in _rows(path):
                if a.kernel in r["Kernel_Name"]:
                    vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
        lines += [""] + [f"{k}_per_dispatch: {statistics.fmean(v):.1f} (n={len(v)})" for k, v in sorted(vals.items())]
        mean = {k: statistics.fmean(v) for k, v in vals.items()}
        if "GRBM_GUI_ACTIVE" in mean:
            # rocprofv3 sums GRBM_GUI_ACTIVE over the XCDs: the kernel's cycles
            # are the sum divided by their number
            cyc = mean["GRBM_GUI_ACTIVE"] / a.xcds
            lines.append(f"gpu_cycles_per_dispatch: {cyc:.1f}  (GRBM_GUI_ACTIVE / {a.xcds} XCDs)")
            if "SQ_VALU_MFMA_BUSY_CYCLES" in mean:
                lines.append(f"mfma_busy_fraction: {mean['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * a.cus * 4):.4f}"
                             f"  (SQ_VALU_MFMA_BUSY_CYCLES / (cycles x {a.cus} CUs x 4 SIMDs))")
        if "SQ_WAVE_CYCLES" in mean and mean["SQ_WAVE_CYCLES"]:
            for k in ("SQ_WAIT_INST_ANY", "SQ_WAIT_ANY", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_VALU", "SQ_ACTIVE_INST_LDS"):
                if k in mean:
                    lines.append(f"{k.lower()}_over_wave_cycles: {mean[k] / mean['SQ_WAVE_CYCLES']:.4f}")
        if "SQ_LDS_BANK_CONFLICT" in mean and "SQ_LDS_IDX_ACTIVE" in mean and mean["SQ_LDS_IDX_ACTIVE"]:
            lines.append(f"lds_bank_conflict_over_active: {mean['SQ_LDS_BANK_CONFLICT'] / mean['SQ_LDS_IDX_ACTIVE']:.4f}")
        if "SQ_INSTS_LDS" in mean and "SQ_VALU_MFMA_BUSY_CYCLES" in mean and mean["SQ_VALU_MFMA_BUSY_CYCLES"]:
            lines.append(f"lds_instructions_per_mfma: {mean['SQ_INSTS_LDS'] * 32 / mean['SQ_VALU_MFMA_BUSY_CYCLES']:.3f}"
                         "  (one 32x32x16 fp16 MFMA = 32 busy cycles)")
    lines += ["", "command:", a.command, ""]
    with open(a.out, "w") as f:
        f.write("\n".join(lines))
    print("\n".join(lines))


def read_field(path, key):
    """Value of ``key:`` in a summary written by this module (None if absent)."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        return None
    return None


if __name__ == "__main__":
    main()
