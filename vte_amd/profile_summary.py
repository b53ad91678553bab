"""Summarise rocprofv3 CSV output of ``bench.py --profile-step`` into the text
kept under profiles/.

    python -m vte_amd.profile_summary stats   <kernel_stats.csv>  <out.md> "<command>" [<kernel substring>]
    python -m vte_amd.profile_summary traffic <fetch counter_collection.csv> <write counter_collection.csv>
                                              <kernel substring> <out.json> <out.md> "<commands>"
    python -m vte_amd.profile_summary mfma    <counter_collection.csv> <out.md> "<command>"
    python -m vte_amd.profile_summary grid    <kernel_trace.csv> <out.md>   (appends a per-launch-shape table)

``traffic``: FETCH_SIZE / WRITE_SIZE are averaged per dispatch of the named
kernel and converted to bytes with the factor that makes the run's 256 MiB
calibration copy (``__amd_rocclr_copyBuffer`` dispatch of that size) read and
write exactly 256 MiB.
"""
from __future__ import annotations

import csv
import json
import sys
from collections import defaultdict

CALIB_BYTES = 256 << 20


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def stats(path, out_md, command, kernel=None):
    rows = _rows(path)
    lines = ["# Kernel trace summary", "", f"Command: `{command}`", "",
             "| kernel | calls | avg us | min us | max us | share % |", "|---|---|---|---|---|---|"]
    for r in rows:
        lines.append(f"| `{r['Name'][:110]}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    if kernel:
        sel = [r for r in rows if kernel in r["Name"]]
        n = sum(int(r["Calls"]) for r in sel)
        tot = sum(float(r["TotalDurationNs"]) for r in sel)
        lines += ["", f"All `{kernel}*` dispatches ({len(sel)} instantiations): {n} calls, "
                  f"average {tot / max(n, 1) / 1e3:.3f} us per launch."]
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")


def _per_kernel(path, counter):
    vals = defaultdict(list)
    for r in _rows(path):
        if r["Counter_Name"] == counter:
            vals[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return vals


def _calibration(vals, expect_kib):
    """Counter KiB of the calibration copy = the largest copyBuffer dispatch."""
    cands = [v for k, vs in vals.items() if "copyBuffer" in k for v in vs]
    if not cands:
        raise SystemExit("no calibration copy dispatch found")
    return expect_kib / max(cands)


def traffic(fetch_csv, write_csv, kernel, out_json, out_md, commands):
    fv, wv = _per_kernel(fetch_csv, "FETCH_SIZE"), _per_kernel(write_csv, "WRITE_SIZE")
    kib = CALIB_BYTES / 1024
    f_scale, w_scale = _calibration(fv, kib), _calibration(wv, kib)
    res = {"kernel": kernel, "fetch_scale": f_scale, "write_scale": w_scale, "per_kernel": {}}
    lines = ["# HBM traffic per dispatch (rocprofv3 counters)", "", "Commands:", ""]
    lines += [f"    {c}" for c in commands.split(" && ")]
    lines += ["", f"Calibration: a 256 MiB device-to-device copy reads/writes 262144 KiB; its FETCH_SIZE "
              f"reads {kib / f_scale:.1f} and WRITE_SIZE {kib / w_scale:.1f}, so counter values are scaled by "
              f"{f_scale:.4f} (fetch) and {w_scale:.4f} (write).", "",
              "| kernel | dispatches | fetch MB/dispatch | write MB/dispatch |", "|---|---|---|---|"]
    for name in sorted(set(fv) | set(wv)):
        f = sum(fv[name]) / max(len(fv[name]), 1) * f_scale * 1024
        w = sum(wv[name]) / max(len(wv[name]), 1) * w_scale * 1024
        res["per_kernel"][name] = {"dispatches": len(fv[name]), "fetch_bytes": f, "write_bytes": w}
        lines.append(f"| `{name[:100]}` | {len(fv[name])} | {f / 1e6:.3f} | {w / 1e6:.3f} |")
    # every instantiation whose name contains ``kernel``, weighted by dispatches
    sel = [k for k in res["per_kernel"] if kernel in k]
    if not sel:
        raise SystemExit(f"kernel {kernel!r} not in the counter output")
    n = sum(res["per_kernel"][k]["dispatches"] for k in sel)
    tot = sum((res["per_kernel"][k]["fetch_bytes"] + res["per_kernel"][k]["write_bytes"])
              * res["per_kernel"][k]["dispatches"] for k in sel)
    res["hbm_bytes_per_launch"] = int(tot / max(n, 1))
    lines += ["", f"`{kernel}*` ({len(sel)} instantiations, {n} dispatches): "
              f"{res['hbm_bytes_per_launch'] / 1e6:.3f} MB of HBM traffic per launch (fetch + write)."]
    with open(out_json, "w") as f:
        json.dump({"kernel": kernel, "instantiations": sel, "dispatches": n,
                   "hbm_bytes_per_launch": res["hbm_bytes_per_launch"],
                   "fetch_scale": f_scale, "write_scale": w_scale}, f, indent=1)
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")


SIMDS = 1024       # MI355X: 256 CUs x 4 SIMDs
GRBM_INSTANCES = 8  # GRBM_GUI_ACTIVE arrives summed over the 8 XCDs


def mfma(path, out_md, command):
    """Per kernel: MFMA work (SQ_INSTS_VALU_MFMA_MOPS_F16 x 512 flops), its
    rate over the dispatch's duration, and MFMA busy share
    SQ_VALU_MFMA_BUSY_CYCLES / (SIMDs x GRBM_GUI_ACTIVE / 8)."""
    per = defaultdict(lambda: defaultdict(float))
    disp = defaultdict(dict)
    for r in _rows(path):
        key = r["Kernel_Name"][:100]
        did = r["Dispatch_Id"]
        per[key][r["Counter_Name"]] += float(r["Counter_Value"])
        disp[key][did] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-9
    lines = ["# MFMA utilisation per kernel", "", f"Command: `{command}`", "",
             "MFMA flops = SQ_INSTS_VALU_MFMA_MOPS_F16 x 512; busy = SQ_VALU_MFMA_BUSY_CYCLES / "
             f"({SIMDS} SIMDs x GRBM_GUI_ACTIVE / {GRBM_INSTANCES}); VALU = SQ_INSTS_VALU per dispatch.", "",
             "| kernel | dispatches | avg us | MFMA GFLOP / dispatch | MFMA TFLOP/s | MFMA busy % | VALU instr / dispatch |",
             "|---|---|---|---|---|---|---|"]
    rows = []
    for key, c in per.items():
        n = len(disp[key])
        t = sum(disp[key].values())
        flops = c.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0) * 512
        if flops == 0:
            continue
        act = c.get("GRBM_GUI_ACTIVE", 0.0) / GRBM_INSTANCES
        busy = 100.0 * c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (SIMDS * act) if act else 0.0
        rows.append((t, f"| `{key}` | {n} | {t / n * 1e6:.2f} | {flops / n / 1e9:.3f} | {flops / t / 1e12:.1f} | "
                        f"{busy:.1f} | {c.get('SQ_INSTS_VALU', 0.0) / n:.3g} |"))
    lines += [r for _, r in sorted(rows, reverse=True)]
    with open(out_md, "w") as f:
        f.write("\n".join(lines) + "\n")


def grid(trace_csv, out_md):
    """Append to out_md the average kernel time per (kernel, grid, workgroup),
    which tells apart launches of one symbol over different matrix shapes."""
    acc = defaultdict(list)
    for r in _rows(trace_csv):
        if r.get("Kind") != "KERNEL_DISPATCH":
            continue
        key = (r["Kernel_Name"], f'{r["Grid_Size_X"]}x{r["Grid_Size_Y"]}', r["Workgroup_Size_X"])
        acc[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    lines = ["", "Per launch shape (grid in threads):", "",
             "| kernel | grid | workgroup | calls | avg us | min us |", "|---|---|---|---|---|---|"]
    for (k, g, w), ts in sorted(acc.items(), key=lambda kv: (kv[0][0], -len(kv[1]))):
        if k.startswith("__amd_rocclr"):
            continue
        lines.append(f"| `{k[:90]}` | {g} | {w} | {len(ts)} | {sum(ts) / len(ts):.2f} | {min(ts):.2f} |")
    with open(out_md, "a") as f:
        f.write("\n".join(lines) + "\n")


if __name__ == "__main__":
    if sys.argv[1] == "stats":
        stats(sys.argv[2], sys.argv[3], sys.argv[4], sys.argv[5] if len(sys.argv) > 5 else None)
    elif sys.argv[1] == "traffic":
        traffic(*sys.argv[2:8])
    elif sys.argv[1] == "mfma":
        mfma(sys.argv[2], sys.argv[3], sys.argv[4])
    elif sys.argv[1] == "grid":
        grid(sys.argv[2], sys.argv[3])
    else:
        raise SystemExit(__doc__)
