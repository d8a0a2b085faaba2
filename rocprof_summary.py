#!/usr/bin/env python3
"""Summarise rocprofv3 result databases (rocpd SQLite) into profiles/.

  trace <db> <out.md> "<command>"
      per-kernel dispatch count and duration statistics (kernel trace).
  traffic <fetch_db> <write_db> <kernel-substring> <out.json> "<fetch cmd>" "<write cmd>"
      mean FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the kernel, and the
      same counters on the 256 MiB device copies bench.py --calibrate runs,
      giving the scale factors bench.py applies (counter KiB / true KiB).
  counters <out.md> <kernel-substring> <db>=<command> [<db>=<command> ...]
      mean value per dispatch of every counter each database holds, for the
      kernels whose name contains the substring.
  mfma <db> <out.md> "<command>"
      MFMA utilisation per kernel from rocprofv3's MfmaUtil and the f16 MFMA
      operation count SQ_INSTS_VALU_MFMA_MOPS_F16.
"""
import json
import sqlite3
import statistics
import sys

CALIB_BYTES = 256 << 20
SIMDS = 256 * 4  # MI355X: 256 CUs x 4 SIMDs


def kernel_rows(db):
    con = sqlite3.connect(db)
    return con.execute("select name, duration from kernels").fetchall()


def short(name):
    """Readable kernel name: the demangled name without its arguments, or,
    for a name the profiler left mangled (_ZN<len><id>...E...), its
    namespace path."""
    if name.startswith("_ZN"):
        parts, i = [], 3
        while i < len(name) and name[i].isdigit():
            j = i
            while name[j].isdigit():
                j += 1
            n = int(name[i:j])
            parts.append(name[j:j + n])
            i = j + n
        if parts:
            return "::".join(p for p in parts if not p.startswith("_GLOBAL__N"))
    return name.replace("(anonymous namespace)::", "").split("(")[0].replace("void ", "")


def trace(db, out, cmd):
    by = {}
    for name, dur in kernel_rows(db):
        by.setdefault(short(name), []).append(dur / 1000.0)
    lines = [f"# Kernel trace: {out.split('/')[-1].rsplit('.', 1)[0]}", "", "Command (GPU box, repo root):", "",
             "```", cmd, "```", "",
             "| kernel | dispatches | mean us | median us | min us | max us | total ms |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    stats = {}
    for k, v in sorted(by.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{k}` | {len(v)} | {statistics.mean(v):.3f} | {statistics.median(v):.3f} | {min(v):.3f} | "
                     f"{max(v):.3f} | {sum(v) / 1000:.3f} |")
        stats[k] = {"dispatches": len(v), "mean_us": statistics.mean(v), "median_us": statistics.median(v)}
    # dispatches that started within 1 us of the previous dispatch's end:
    # the graph replays (and launch loops the host kept ahead of), which is
    # where bench.py's value is measured; the others ran after the GPU had
    # idled (eager calls from Python, host-buffer calls)
    con = sqlite3.connect(db)
    seq = con.execute("select name, start, end from kernels order by start").fetchall()
    b2b = {}
    for (_, _, pe), (name, st, en) in zip(seq, seq[1:]):
        if st - pe < 1000:
            b2b.setdefault(short(name), []).append((en - st) / 1000.0)
    if b2b:
        lines += ["", "Back-to-back dispatches only (start within 1 us of the previous dispatch's end: graph replays):",
                  "", "| kernel | dispatches | mean us | median us | min us | max us |", "|---|---:|---:|---:|---:|---:|"]
        for k, v in sorted(b2b.items(), key=lambda kv: -sum(kv[1])):
            lines.append(f"| `{k}` | {len(v)} | {statistics.mean(v):.3f} | {statistics.median(v):.3f} | "
                         f"{min(v):.3f} | {max(v):.3f} |")
            stats.setdefault(k, {})["back_to_back_mean_us"] = statistics.mean(v)
    open(out, "w").write("\n".join(lines) + "\n")
    return stats


def pmc_values(db, counter):
    con = sqlite3.connect(db)
    rows = con.execute("select kernel_name, grid_size, value from counters_collection where counter_name = ?",
                       (counter,)).fetchall()
    return rows


def traffic(fetch_db, write_db, kernel, out, fetch_cmd, write_cmd):
    res = {"dominant": kernel, "kernels": {}, "copy_calibration": {}, "commands": [fetch_cmd, write_cmd]}
    for db, counter in ((fetch_db, "FETCH_SIZE"), (write_db, "WRITE_SIZE")):
        rows = pmc_values(db, counter)
        by = {}
        for name, grid, val in rows:
            by.setdefault(short(name), []).append(val)
        for k, v in by.items():
            res["kernels"].setdefault(k, {})[f"{counter}_kib"] = statistics.mean(v)
            res["kernels"][k]["dispatches"] = len(v)
        # calibration: the largest copyBuffer dispatches are the 256 MiB copies
        copies = sorted((val for name, grid, val in rows if "copyBuffer" in name), reverse=True)[:3]
        factor = statistics.mean(copies) / (CALIB_BYTES / 1024.0) if copies else None
        res["copy_calibration"]["fetch_factor" if counter == "FETCH_SIZE" else "write_factor"] = factor
        res["copy_calibration"][f"{counter}_kib_per_256MiB_copy"] = copies
    match = [k for k in res["kernels"] if kernel in k]
    if match:
        res["dominant"] = match[0]
    json.dump(res, open(out, "w"), indent=1)
    md = out.rsplit(".", 1)[0] + ".md"
    d = res["kernels"].get(res["dominant"], {})
    cal = res["copy_calibration"]
    f_kib, w_kib = d.get("FETCH_SIZE_kib"), d.get("WRITE_SIZE_kib")
    lines = [f"# HBM traffic: {res['dominant']}", "", "Commands (GPU box, repo root):", "", "```", fetch_cmd,
             write_cmd, "```", "",
             f"- FETCH_SIZE per dispatch: {f_kib:.1f} KiB (mean of {d.get('dispatches')} dispatches)" if f_kib else
             "- FETCH_SIZE: n/a",
             f"- WRITE_SIZE per dispatch: {w_kib:.1f} KiB" if w_kib else "- WRITE_SIZE: n/a",
             f"- copy calibration (256 MiB device copy): FETCH factor {cal.get('fetch_factor')}, "
             f"WRITE factor {cal.get('write_factor')}",
             ]
    if f_kib and w_kib and cal.get("fetch_factor") and cal.get("write_factor"):
        tb = (f_kib / cal["fetch_factor"] + w_kib / cal["write_factor"]) * 1024
        lines.append(f"- HBM bytes per dispatch (scaled): {tb:,.0f} B")
        res["hbm_bytes_per_dispatch"] = tb
        json.dump(res, open(out, "w"), indent=1)
    lines += ["", "| kernel | FETCH KiB/dispatch | WRITE KiB/dispatch |", "|---|---:|---:|"]
    for k, v in res["kernels"].items():
        lines.append(f"| `{k}` | {v.get('FETCH_SIZE_kib', float('nan')):.1f} | {v.get('WRITE_SIZE_kib', float('nan')):.1f} |")
    open(md, "w").write("\n".join(lines) + "\n")


def mfma(db, out, cmd):
    """rocprofv3's derived counter MfmaUtil (= sum of SQ_VALU_MFMA_BUSY_CYCLES
    / (max GRBM_GUI_ACTIVE x SIMDs) x 100) and the f16 MFMA FLOPs
    (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512), per kernel."""
    con = sqlite3.connect(db)
    rows = con.execute("select dispatch_id, kernel_name, counter_name, value from counters_collection").fetchall()
    per = {}
    for did, name, cname, val in rows:
        d = per.setdefault((did, short(name)), {})
        d[cname] = d.get(cname, 0.0) + val  # derived counters: one row per dispatch
    by = {}
    for (did, name), c in per.items():
        by.setdefault(name, []).append(c)
    lines = ["# MFMA utilisation: batched prefill (config 5)", "", "Command (GPU box, repo root):", "", "```", cmd,
             "```", "",
             "MfmaUtil (rocprofv3 derived counter) = sum over the GPU of SQ_VALU_MFMA_BUSY_CYCLES / (max",
             "GRBM_GUI_ACTIVE x SIMDs) x 100; f16 MFMA FLOPs = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 (f16 MFMA FLOPs",
             "issued, padding rows included).", "",
             "| kernel | dispatches | mean MfmaUtil % | mean f16 MFMA GFLOP |", "|---|---:|---:|---:|"]
    for k, v in sorted(by.items()):
        util = [c["MfmaUtil"] for c in v if "MfmaUtil" in c]
        fl = [c["SQ_INSTS_VALU_MFMA_MOPS_F16"] * 512 for c in v if "SQ_INSTS_VALU_MFMA_MOPS_F16" in c]
        if not util:
            continue
        lines.append(f"| `{k}` | {len(v)} | {statistics.mean(util):.2f} | "
                     f"{statistics.mean(fl) / 1e9 if fl else float('nan'):.2f} |")
    open(out, "w").write("\n".join(lines) + "\n")


def counters(out, kernel, pairs):
    rows = {}
    cmds = []
    for pair in pairs:
        db, cmd = pair.split("=", 1)
        cmds.append(cmd)
        con = sqlite3.connect(db)
        for name, cname, val in con.execute("select kernel_name, counter_name, value from counters_collection"):
            k = short(name)
            if kernel in k:
                rows.setdefault((k, cname), []).append(val)
    lines = [f"# Counters: {out.split('/')[-1].rsplit('.', 1)[0]}", "", "Commands (GPU box, repo root):", "", "```"]
    lines += cmds + ["```", "", "Mean per dispatch (rocprofv3's aggregation over the GPU).", "",
                     "| kernel | counter | dispatches | mean |", "|---|---|---:|---:|"]
    for (k, c), v in sorted(rows.items()):
        lines.append(f"| `{k}` | {c} | {len(v)} | {statistics.mean(v):,.0f} |")
    open(out, "w").write("\n".join(lines) + "\n")


if __name__ == "__main__":
    mode = sys.argv[1]
    if mode == "trace":
        trace(*sys.argv[2:5])
    elif mode == "traffic":
        traffic(*sys.argv[2:8])
    elif mode == "counters":
        counters(sys.argv[2], sys.argv[3], sys.argv[4:])
    elif mode == "mfma":
        mfma(*sys.argv[2:5])
    else:
        sys.exit(__doc__)
