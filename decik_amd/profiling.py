"""Summaries of rocprofv3 output for the kernels of this package (the text under profiles/).

rocprofv3 writes CSV files with --output-format csv: <prefix>_kernel_stats.csv and
<prefix>_kernel_trace.csv for --kernel-trace --stats, <prefix>_counter_collection.csv for --pmc.
This module reduces them to short markdown tables (or, for the traffic of one launch, JSON):

  python -m decik_amd.profiling trace <dir> <prefix> --title T --command C [--match RE]
  python -m decik_amd.profiling counters <dir> <prefix> --title T --command C [--match RE]
  python -m decik_amd.profiling traffic <fetch_dir> <write_dir> <prefix> --match RE --command C --command C
  python -m decik_amd.profiling traffic-table <fetch_dir:write_dir:prefix:label> ... --title T --command C ...

`trace`: rocprofv3's own per-kernel totals, then every matching kernel by launch shape (grid):
launches, median / mean / min duration, VGPRs, LDS. `counters`: per kernel and grid the mean of
each counter over its dispatches and the usual ratios (VALU and LDS instructions per MFMA, MFMA
busy share, wait share). `traffic`: HBM bytes per dispatch of the launch matched by RE (its most
frequent kernel and grid, plus the split-K reduction dispatched right after it) from FETCH_SIZE
and WRITE_SIZE, each scaled by what the counter reads for the fp32 -> fp16 conversion of 128 Mi
values that bench.py --copy-probe runs (512 MiB read, 256 MiB written). `traffic-table`: the same
scaled bytes for every matching kernel and grid of several pass pairs, as a markdown table.
"""

import argparse
import collections
import csv
import json
import os
import re
import statistics
import sys


def _rows(run_dir, prefix, kind):
    path = os.path.join(run_dir, f"{prefix}_{kind}.csv")
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def _short(name, n=90):
    return name if len(name) <= n else name[: n - 3] + "..."


def trace_summary(run_dir, prefix, title, command, match=r"dk::", top=12):
    stats = _rows(run_dir, prefix, "kernel_stats")
    trace = _rows(run_dir, prefix, "kernel_trace")
    out = [f"# rocprofv3 kernel trace: {title}", "", "Command (from /tmp, TMPDIR=/tmp):", "", "```", command, "```", "",
           "## Per-kernel totals (rocprofv3 --stats, top entries)", "",
           "| kernel | calls | avg us | total % |", "|---|---:|---:|---:|"]
    for r in stats[:top]:
        out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['Percentage']):.2f} |")
    out += ["", "## Matching kernels by launch shape (kernel trace)", "",
            "| kernel | grid (threads) | launches | median us | mean us | min us | VGPRs | LDS bytes |",
            "|---|---:|---:|---:|---:|---:|---:|---:|"]
    rx = re.compile(match)
    groups, meta, order = collections.defaultdict(list), {}, []
    for r in trace:
        name = r["Kernel_Name"]
        if not rx.search(name):
            continue
        key = (name, r.get("Grid_Size_X") or r.get("Grid_Size"))
        if key not in groups:
            order.append(key)
        groups[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        meta[key] = (r.get("VGPR_Count", ""), r.get("LDS_Block_Size", ""))
    for key in order:
        v = groups[key]
        out.append(f"| `{_short(key[0], 70)}` | {key[1]} | {len(v)} | {statistics.median(v):.2f} | "
                   f"{statistics.fmean(v):.2f} | {min(v):.2f} | {meta[key][0]} | {meta[key][1]} |")
    return "\n".join(out) + "\n"


def _counter_means(rows, match):
    rx = re.compile(match)
    acc = collections.defaultdict(lambda: collections.defaultdict(list))
    order = []
    for r in rows:
        if not rx.search(r["Kernel_Name"]):
            continue
        key = (r["Kernel_Name"], r.get("Grid_Size") or r.get("Grid_Size_X"))
        if key not in acc:
            order.append(key)
        acc[key][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return order, {k: {c: statistics.fmean(v) for c, v in d.items()} for k, d in acc.items()}


def counter_summary(run_dirs_prefixes, title, commands, match=r"dk::"):
    order, means = [], {}
    for run_dir, prefix in run_dirs_prefixes:
        o, m = _counter_means(_rows(run_dir, prefix, "counter_collection"), match)
        for k in o:
            if k not in means:
                order.append(k)
                means[k] = {}
            means[k].update(m[k])
    out = [f"# rocprofv3 counters: {title}", "", "Commands (from /tmp, TMPDIR=/tmp; one pass each):", "", "```"]
    out += list(commands) + ["```", "", "Means per dispatch over every dispatch of the kernel and grid in the run, "
                                        "summed over the whole device.", ""]
    ratio_cols = [("VALU/MFMA", "SQ_INSTS_VALU", "SQ_INSTS_MFMA"), ("LDS/MFMA", "SQ_INSTS_LDS", "SQ_INSTS_MFMA"),
                  ("MFMA busy / SIMD-cycles", "SQ_VALU_MFMA_BUSY_CYCLES", None),
                  ("wait / wave-cycles", "SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES")]
    out += ["| kernel | grid | " + " | ".join(c[0] for c in ratio_cols) + " |",
            "|---|---:|" + "---:|" * len(ratio_cols)]
    for key in order:
        m = means[key]
        cells = []
        for _, num, den in ratio_cols:
            if num not in m:
                cells.append("-")
            elif den is None:
                # SIMD-cycles of the dispatch: GRBM_GUI_ACTIVE (summed over the 8 XCDs) / 8 x 1024 SIMDs
                cells.append(f"{m[num] / (m['GRBM_GUI_ACTIVE'] / 8 * 1024):.3f}" if "GRBM_GUI_ACTIVE" in m else "-")
            else:
                cells.append(f"{m[num] / m[den]:.2f}" if m.get(den) else "-")
        out.append(f"| `{_short(key[0], 60)}` | {key[1]} | " + " | ".join(cells) + " |")
    names = sorted({c for m in means.values() for c in m})
    out += ["", "Raw means per dispatch:", "", "| counter | " + " | ".join(f"`{_short(k[0], 40)}` {k[1]}" for k in order) + " |",
            "|---|" + "---:|" * len(order)]
    for c in names:
        out.append(f"| {c} | " + " | ".join(f"{means[k].get(c, float('nan')):.0f}" for k in order) + " |")
    return "\n".join(out) + "\n"


def traffic(fetch_dir, write_dir, prefix, match, commands, launch=None, plan=None, commit=None):
    def load(run_dir):
        rows = sorted(_rows(run_dir, prefix, "counter_collection"), key=lambda r: int(r["Dispatch_Id"]))
        rx = re.compile(match)
        cnt = collections.Counter((r["Kernel_Name"], int(r["Grid_Size"])) for r in rows if rx.search(r["Kernel_Name"]))
        main = cnt.most_common(1)[0][0]
        per, prev = collections.defaultdict(list), None
        for r in rows:
            key = (r["Kernel_Name"], int(r["Grid_Size"]))
            # a split-K reduction belongs to this launch only right after its GEMM kernel
            if "splitk_reduce_kernel" in key[0] and prev != main:
                prev = key
                continue
            per[key].append(float(r["Counter_Value"]))
            prev = key
        return per, main

    (fetch, main), (write, _) = load(fetch_dir), load(write_dir)
    cal = max((k for k in fetch if "float16_copy" in k[0]), key=lambda k: max(fetch[k]))
    cal_f, cal_w = max(fetch[cal]), max(write[cal])
    sf, sw = (512 * 1024) / cal_f, (256 * 1024) / cal_w
    parts = [main] + [k for k in fetch if "splitk_reduce_kernel" in k[0] and k in write]
    detail, total = [], 0.0
    for k in parts:
        f, w = statistics.fmean(fetch[k]), statistics.fmean(write[k])
        b = f * 1024 * sf + w * 1024 * sw
        total += b
        detail.append(dict(kernel=_short(k[0], 80), grid=k[1], dispatches=len(fetch[k]), fetch_kib_raw=round(f, 1),
                           write_kib_raw=round(w, 1), bytes=round(b)))
    return dict(note="HBM bytes per call of one launch: FETCH_SIZE and WRITE_SIZE (KiB per dispatch, mean over "
                     "the dispatches) of its kernels, scaled so that the fp32->fp16 conversion of 128 Mi values "
                     "reads 512 MiB and writes 256 MiB",
                launch=launch, plan=plan, commit=commit, match=match, bytes_per_call=round(total), kernels=detail,
                commands=list(commands),
                calibration=dict(kernel=_short(cal[0], 100), fetch_kib=cal_f, write_kib=cal_w,
                                 fetch_scale=round(sf, 4), write_scale=round(sw, 4)))


def traffic_table(runs, title, commands, match):
    """Markdown table of HBM bytes per dispatch of every (kernel, grid) matching `match` in
    several FETCH_SIZE / WRITE_SIZE pass pairs (runs: (fetch_dir, write_dir, prefix, label)), each
    pass scaled by its own fp32 -> fp16 conversion probe (bench.py --copy-probe)."""
    out = [f"# rocprofv3 HBM traffic: {title}", "", "Commands (from /tmp, TMPDIR=/tmp; one pass each):", "", "```"]
    out += list(commands) + ["```", "",
                             "Bytes per dispatch: FETCH_SIZE and WRITE_SIZE (KiB, mean over the dispatches of "
                             "the kernel and grid), scaled so that the fp32 -> fp16 conversion of 128 Mi values "
                             "reads 512 MiB and writes 256 MiB.", "",
                             "| run | kernel | grid | dispatches | read MB | written MB | total MB |",
                             "|---|---|---:|---:|---:|---:|---:|"]
    rx = re.compile(match)
    for fetch_dir, write_dir, prefix, label in runs:
        per = []
        for d in (fetch_dir, write_dir):
            acc = collections.defaultdict(list)
            for r in _rows(d, prefix, "counter_collection"):
                acc[(r["Kernel_Name"], int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
            per.append(acc)
        fetch, write = per
        cal = max((k for k in fetch if "float16_copy" in k[0]), key=lambda k: max(fetch[k]))
        sf, sw = (512 * 1024) / max(fetch[cal]), (256 * 1024) / max(write[cal])
        for k in sorted(fetch, key=lambda k: (k[0], k[1])):
            if not rx.search(k[0]) or k not in write:
                continue
            f = statistics.fmean(fetch[k]) * 1024 * sf / 1e6
            w = statistics.fmean(write[k]) * 1024 * sw / 1e6
            out.append(f"| {label} | `{_short(k[0], 60)}` | {k[1]} | {len(fetch[k])} | {f:.2f} | {w:.2f} | {f + w:.2f} |")
    return "\n".join(out) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(prog="python -m decik_amd.profiling")
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("dir")
    t.add_argument("prefix")
    t.add_argument("--title", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--match", default=r"dk::")
    c = sub.add_parser("counters")
    c.add_argument("runs", nargs="+", help="dir:prefix of each --pmc pass")
    c.add_argument("--title", required=True)
    c.add_argument("--command", action="append", required=True)
    c.add_argument("--match", default=r"dk::")
    f = sub.add_parser("traffic")
    f.add_argument("fetch_dir")
    f.add_argument("write_dir")
    f.add_argument("prefix")
    f.add_argument("--match", required=True)
    f.add_argument("--command", action="append", required=True)
    f.add_argument("--launch", default=None, help="the launch kind bench.py names (its roofline reads the file)")
    f.add_argument("--plan", default=None,
                   help="JSON of the launch plan the counters were taken on (bench.py's mlp_plan(launch)): "
                        "bench.py ignores the file once the planner picks another plan")
    f.add_argument("--commit", default=None, help="the commit the counters were taken on")
    tt = sub.add_parser("traffic-table")
    tt.add_argument("runs", nargs="+", help="fetch_dir:write_dir:prefix:label of each pass pair")
    tt.add_argument("--title", required=True)
    tt.add_argument("--command", action="append", required=True)
    tt.add_argument("--match", default=r"dk::")
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        sys.stdout.write(trace_summary(a.dir, a.prefix, a.title, a.command, a.match))
    elif a.cmd == "traffic-table":
        sys.stdout.write(traffic_table([tuple(r.split(":", 3)) for r in a.runs], a.title, a.command, a.match))
    elif a.cmd == "counters":
        runs = [tuple(r.rsplit(":", 1)) for r in a.runs]
        sys.stdout.write(counter_summary(runs, a.title, a.command, a.match))
    else:
        plan = json.loads(a.plan) if a.plan else None
        json.dump(traffic(a.fetch_dir, a.write_dir, a.prefix, a.match, a.command, a.launch, plan, a.commit),
                  sys.stdout, indent=1)
        sys.stdout.write("\n")


if __name__ == "__main__":
    main()
