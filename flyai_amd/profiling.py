"""Summaries of rocprofv3 CSV output (``-f csv``) for the stage step and the MXFP4 expert kernels.

Two reports, both plain text for committing beside the numbers they support:

* ``stats``: the ``--kernel-trace --stats`` kernel table of a ``bench.py`` run, plus the average
  duration of the last ``reps`` dispatches of one kernel (the isolated launches ``bench.py`` times
  with HIP events after the stage steps);
* ``traffic``: HBM bytes per launch of one kernel from two ``--pmc`` runs (``FETCH_SIZE`` and
  ``WRITE_SIZE``, KiB per dispatch).  Each reading is scaled by the reading of a plain device copy
  of known size in the same run (``bench.py --copy-probe-mib M``): factor = M MiB / copy reading.

* ``collect``: runs the kernel trace and the counter passes (PMC_PASSES) of one ``bench.py``
  workload under rocprofv3, as child processes, and writes both reports for it;
* ``counters``: per (kernel, grid size) the mean of every counter of one or more ``--pmc`` runs
  (HBM bytes through the same copy calibration, unit busy/stall cycles as a fraction of the CUs'
  cycles, MFMA ops as TFLOP/s) beside the mean duration from a ``--kernel-trace`` run.

Usage::

    python -m flyai_amd.profiling collect --name c2 OUT -- --workload c2     (on the GPU machine)

    python -m flyai_amd.profiling stats DIR --kernel moe_mxfp4_kernel<true --reps 50 --command "..."
    python -m flyai_amd.profiling traffic FETCH_DIR WRITE_DIR --kernel moe_mxfp4_kernel<true \\
        --reps 5 --copy-mib 256 --json OUT.json --command-fetch "..." --command-write "..."
"""
import argparse
import csv
import glob
import json
import os
import sys


def _find(dirname, suffix):
    hits = sorted(glob.glob(os.path.join(dirname, "**", "*" + suffix), recursive=True))
    if not hits:
        raise FileNotFoundError(f"no *{suffix} under {dirname}")
    return hits[-1]


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def short_name(name):
    n = name.replace("void ", "").replace("flyai::", "").replace("(anonymous namespace)::", "")
    depth, out = 0, []
    for ch in n:           # drop the parameter list, keep template arguments
        if ch == "(" and depth == 0:
            break
        depth += ch == "<"
        depth -= ch == ">"
        out.append(ch)
    n = "".join(out).strip()
    return n if len(n) <= 96 else n[:93] + "..."


def kernel_table(dirname, top=24):
    rows = _rows(_find(dirname, "kernel_stats.csv"))
    total = sum(float(r["TotalDurationNs"]) for r in rows)
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    lines = ["| kernel | calls | avg us | min us | max us | total ms | % |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for r in rows[:top]:
        lines.append(f"| `{short_name(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | "
                     f"{float(r['TotalDurationNs']) / 1e6:.3f} | {100 * float(r['TotalDurationNs']) / total:.1f} |")
    return lines, total


def last_dispatches(dirname, kernel, reps):
    """(Dispatch_Id, duration ns) of the last ``reps`` dispatches whose name contains ``kernel``."""
    rows = [r for r in _rows(_find(dirname, "kernel_trace.csv")) if kernel in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    return [(int(r["Dispatch_Id"]), int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) for r in rows[-reps:]]


def counter_by_dispatch(dirname, counter):
    """{Dispatch_Id: (kernel name, summed value)} for one counter."""
    out = {}
    for r in _rows(_find(dirname, "counter_collection.csv")):
        if r["Counter_Name"] != counter:
            continue
        d = int(r["Dispatch_Id"])
        name, v = out.get(d, (r["Kernel_Name"], 0.0))
        out[d] = (name, v + float(r["Counter_Value"]))
    return out


def _avg_last(by_disp, match, reps):
    ds = sorted(d for d, (name, _) in by_disp.items() if match(name))[-reps:]
    if not ds:
        raise ValueError("no matching dispatches")
    return sum(by_disp[d][1] for d in ds) / len(ds), len(ds)


def traffic(fetch_dir, write_dir, kernel, reps, copy_mib):
    is_copy = lambda n: "copy" in n.lower() and "moe" not in n.lower()
    is_k = lambda n: kernel in n
    copy_kib = copy_mib * 1024.0
    res = {}
    for tag, d, counter in (("read", fetch_dir, "FETCH_SIZE"), ("write", write_dir, "WRITE_SIZE")):
        by = counter_by_dispatch(d, counter)
        k_kib, nk = _avg_last(by, is_k, reps)
        c_kib, nc = _avg_last(by, is_copy, 3)
        factor = copy_kib / c_kib
        res[tag] = {"counter": counter, "kernel_kib": k_kib, "kernel_dispatches": nk,
                    "copy_kib": c_kib, "copy_dispatches": nc, "factor": factor,
                    "bytes": k_kib * factor * 1024.0}
    res["hbm_bytes_per_launch"] = int(round(res["read"]["bytes"] + res["write"]["bytes"]))
    return res


def _grid(r):
    if r.get("Grid_Size"):
        return int(float(r["Grid_Size"]))
    return (int(float(r.get("Grid_Size_X") or 0)) * int(float(r.get("Grid_Size_Y") or 1)) *
            int(float(r.get("Grid_Size_Z") or 1)))


def dispatch_counters(dirname):
    """{Dispatch_Id: (short kernel name, grid size, {counter: (sum, max) over its instance rows})} of
    one ``--pmc`` run."""
    out = {}
    for r in _rows(_find(dirname, "counter_collection.csv")):
        d = int(r["Dispatch_Id"])
        if d not in out:
            out[d] = (short_name(r["Kernel_Name"]), _grid(r), {})
        vals = out[d][2]
        v = float(r["Counter_Value"])
        s, m = vals.get(r["Counter_Name"], (0.0, float("-inf")))
        vals[r["Counter_Name"]] = (s + v, max(m, v))
    return out


def trace_durations(dirname):
    """{(short kernel name, grid size): [duration ns, ...]} of a ``--kernel-trace`` run."""
    out = {}
    for r in _rows(_find(dirname, "kernel_trace.csv")):
        key = (short_name(r["Kernel_Name"]), _grid(r))
        out.setdefault(key, []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    return out


def _copy_factor(disp, counter, copy_mib):
    """Bytes per counter KiB: the last 3 plain-copy dispatches of the run moved copy_mib MiB each."""
    ds = sorted(d for d, (n, _, v) in disp.items() if "copyBuffer" in n and counter in v)[-3:]
    if not ds or copy_mib <= 0:
        return None
    kib = sum(disp[d][2][counter][0] for d in ds) / len(ds)
    return copy_mib * 1024.0 / kib * 1024.0


def counter_table(pmc_dirs, trace_dir, match, copy_mib, n_cu):
    """Per (kernel, grid) whose name contains one of ``match``: dispatch count and mean duration from
    the trace run, and the mean per-dispatch value of every counter of the pmc runs.  FETCH_SIZE and
    WRITE_SIZE become bytes through the copy calibration; *_sum cycle counters become a fraction of
    n_cu x the dispatch's GRBM_GUI_ACTIVE (its busy cycles, the max over XCDs) when that counter was
    read in the same pass; MFMA op counters become TFLOP/s over the trace duration."""
    durs = trace_durations(trace_dir)
    rows = {}
    for d in pmc_dirs:
        disp = dispatch_counters(d)
        factors = {c: _copy_factor(disp, c, copy_mib) for c in ("FETCH_SIZE", "WRITE_SIZE")}
        for _, (name, grid, vals) in disp.items():
            if not any(m in name for m in match):
                continue
            row = rows.setdefault((name, grid), {})
            gui = vals.get("GRBM_GUI_ACTIVE", (0.0, 0.0))[1]
            for c, (s, _) in vals.items():
                if c in factors and factors[c]:
                    row.setdefault(c + "_bytes", []).append(s * factors[c])
                elif c.endswith("_sum") and ("CYCLES" in c or "BUSY" in c) and gui > 0:
                    row.setdefault(c + "_frac", []).append(s / (n_cu * gui))
                elif c.startswith("SQ_INSTS_VALU_MFMA_MOPS"):
                    row.setdefault(c, []).append(s * 512.0)
                elif c != "GRBM_GUI_ACTIVE":
                    row.setdefault(c, []).append(s)
    out = []
    for (name, grid), row in sorted(rows.items()):
        ds = durs.get((name, grid), [])
        ent = {"kernel": name, "grid": grid, "calls": len(ds),
               "avg_us": (sum(ds) / len(ds) / 1e3) if ds else None}
        for c, v in row.items():
            ent[c] = sum(v) / len(v)
        wave_cyc = ent.get("SQ_WAVE_CYCLES")
        if wave_cyc:
            for c, k in (("SQ_WAIT_INST_LDS", "lds_issue_wait_frac"), ("SQ_WAIT_ANY", "wait_any_frac")):
                if c in ent:
                    ent[k] = ent[c] / wave_cyc
        if ent["avg_us"]:
            by = ent.get("FETCH_SIZE_bytes", 0.0) + ent.get("WRITE_SIZE_bytes", 0.0)
            if by:
                ent["hbm_GBps"] = by / (ent["avg_us"] * 1e-6) / 1e9
            fl = sum(v for c, v in ent.items() if c.startswith("SQ_INSTS_VALU_MFMA_MOPS"))
            if fl:
                ent["mfma_TFLOPs"] = fl / (ent["avg_us"] * 1e-6) / 1e12
        out.append(ent)
    return out


def counter_markdown(ents, title, commands):
    cols = [("calls", "calls", "{:.0f}"), ("avg_us", "avg us", "{:.2f}"),
            ("FETCH_SIZE_bytes", "HBM read MB", "{:.2f}"), ("WRITE_SIZE_bytes", "HBM write MB", "{:.2f}"),
            ("hbm_GBps", "HBM GB/s", "{:.0f}"), ("TA_TA_BUSY_sum_frac", "TA busy", "{:.0%}"),
            ("TCP_PENDING_STALL_CYCLES_sum_frac", "L1 pending stall", "{:.0%}"),
            ("TCP_TCC_READ_REQ_sum", "L1->L2 reads", "{:.3g}"), ("MfmaUtil", "MfmaUtil %", "{:.1f}"),
            ("mfma_TFLOPs", "MFMA TFLOP/s", "{:.0f}"), ("LdsUtil", "LdsUtil %", "{:.1f}"),
            ("SQ_LDS_BANK_CONFLICT", "LDS conflict cyc", "{:.3g}"),
            ("lds_issue_wait_frac", "LDS issue wait", "{:.0%}"), ("wait_any_frac", "waiting", "{:.0%}")]
    cols = [c for c in cols if any(c[0] in e and e[c[0]] is not None for e in ents)]
    scale = {"FETCH_SIZE_bytes": 1e-6, "WRITE_SIZE_bytes": 1e-6}
    lines = [f"# {title}", "", "Commands (repo root, ``cd /tmp && export TMPDIR=/tmp`` first):", ""]
    lines += ["    " + c for c in commands]
    lines += ["", "| kernel | grid | " + " | ".join(h for _, h, _ in cols) + " |",
              "|---|---:|" + "---:|" * len(cols)]
    for e in ents:
        cells = []
        for k, _, f in cols:
            v = e.get(k)
            cells.append("" if v is None else f.format(v * scale.get(k, 1.0)))
        lines.append(f"| `{e['kernel']}` | {e['grid']} | " + " | ".join(cells) + " |")
    return lines


# Counter passes of ``collect``: each pass stays within one rocprofv3 run's hardware limits (at most
# 8 SQ, 4 TCC, 4 TCP, 2 TA and 2 GRBM counters).
PMC_PASSES = (
    ("FETCH_SIZE",),
    ("WRITE_SIZE",),
    ("TA_TA_BUSY_sum", "TCP_PENDING_STALL_CYCLES_sum", "TCP_TCC_READ_REQ_sum", "GRBM_GUI_ACTIVE"),
    ("MfmaUtil", "SQ_INSTS_VALU_MFMA_MOPS_BF16", "SQ_INSTS_VALU_MFMA_MOPS_F8", "SQ_INSTS_VALU_MFMA_MOPS_F6F4"),
    ("LdsUtil", "SQ_LDS_BANK_CONFLICT", "SQ_WAIT_INST_LDS", "SQ_WAIT_ANY", "SQ_WAVE_CYCLES"),
)
STAGE_KERNELS = ("moe_", "attn_", "gemm_", "rmsnorm", "qkv_", "pack_", "act_quant", "route", "router",
                 "combine", "mx_", "fp8", "linear_", "grouped_")
# bench.py arguments of the counter passes: few steps, a 256 MiB copy for the byte calibration
PMC_BENCH = ("--no-cpu", "--steps", "2", "--warmup", "1", "--kernel-reps", "5", "--moe-reps", "5",
             "--read-probe-mib", "0", "--copy-probe-mib", "256")


def _run(cmd, log, timeout):
    import subprocess
    with open(log, "w") as f:
        f.write(" ".join(cmd) + "\n")
        f.flush()
        subprocess.run(cmd, stdout=f, stderr=subprocess.STDOUT, timeout=timeout, check=True)


def collect(out, name, bench_args, python=None, timeout=300):
    """Kernel trace + the PMC_PASSES counter passes of ``bench.py bench_args`` under rocprofv3, each a
    child process (this process never touches the GPU), then the counter table (``name_counters.md``
    and ``.json``) and the kernel table (``name_kernel_stats.md``).  Raw rocprofv3 output is removed;
    the kernel trace is kept gzipped.  The program after rocprofv3's ``--`` is the interpreter binary
    itself (this process's, symlinks resolved), so no launcher or shim runs between the profiler's
    preloaded library and bench.py."""
    import gzip
    import shutil
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    bench = [python or os.path.realpath(sys.executable), os.path.join(root, "bench.py")]
    os.makedirs(out, exist_ok=True)
    trace = os.path.join(out, name + "_trace")
    cmds = [["rocprofv3", "--kernel-trace", "--stats", "-f", "csv", "-d", trace, "-o", "run", "--", *bench,
             "--no-cpu", "--read-probe-mib", "0", *bench_args]]
    pmc_dirs = []
    for i, ctrs in enumerate(PMC_PASSES):
        d = os.path.join(out, f"{name}_pmc{i + 1}")
        pmc_dirs.append(d)
        cmds.append(["rocprofv3", "--kernel-trace", "--pmc", *ctrs, "-f", "csv", "-d", d, "-o", "run", "--",
                     *bench, *PMC_BENCH, *bench_args])
    for i, cmd in enumerate(cmds):
        print(f"[profiling] {name} pass {i + 1}/{len(cmds)}", flush=True)
        _run(cmd, os.path.join(out, f"{name}_pass{i + 1}.log"), timeout)
    shown = [" ".join(["python3 -m flyai_amd.profiling collect --name", name, out, "--", *bench_args]),
             "which runs:"] + [" ".join(c) for c in cmds]
    shown = [c.replace(root + os.sep, "") for c in shown]
    ents = counter_table(pmc_dirs, trace, STAGE_KERNELS, 256, 256)
    with open(os.path.join(out, name + "_counters.json"), "w") as f:
        json.dump(ents, f, indent=1)
    with open(os.path.join(out, name + "_counters.md"), "w") as f:
        f.write("\n".join(counter_markdown(ents, f"{name}: per-kernel counters", shown)) + "\n")
    lines, total = kernel_table(trace)
    with open(os.path.join(out, name + "_kernel_stats.md"), "w") as f:
        f.write(f"# {name}: kernel time\n\nCommand (the trace pass of ``{shown[0]}``):\n\n    {shown[2]}\n\n"
                f"All dispatches of the run, total "
                f"{total / 1e6:.3f} ms of kernel time.\n\n" + "\n".join(lines) + "\n")
    with open(_find(trace, "kernel_trace.csv"), "rb") as src, \
            gzip.open(os.path.join(out, name + "_kernel_trace.csv.gz"), "wb") as dst:
        shutil.copyfileobj(src, dst)
    for d in [trace, *pmc_dirs]:
        shutil.rmtree(d, ignore_errors=True)
    return ents


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--kernel", required=True)
    s.add_argument("--reps", type=int, required=True)
    s.add_argument("--command", required=True)
    s.add_argument("--title", default="stage step kernels")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_dir")
    t.add_argument("write_dir")
    t.add_argument("--kernel", required=True)
    t.add_argument("--reps", type=int, required=True)
    t.add_argument("--copy-mib", type=int, required=True)
    t.add_argument("--json", required=True)
    t.add_argument("--command-fetch", required=True)
    t.add_argument("--command-write", required=True)
    c = sub.add_parser("counters")
    c.add_argument("trace_dir")
    c.add_argument("pmc_dirs", nargs="+")
    c.add_argument("--match", action="append", required=True)
    c.add_argument("--copy-mib", type=int, default=0)
    c.add_argument("--cus", type=int, default=256)
    c.add_argument("--title", required=True)
    c.add_argument("--command", action="append", required=True)
    c.add_argument("--json")
    k = sub.add_parser("collect")
    k.add_argument("out")
    k.add_argument("--name", required=True)
    k.add_argument("--timeout", type=int, default=300)
    k.add_argument("bench_args", nargs=argparse.REMAINDER)
    a = ap.parse_args(argv)

    if a.cmd == "collect":
        extra = [x for x in a.bench_args if x != "--"]
        collect(a.out, a.name, extra, timeout=a.timeout)
        return 0
    if a.cmd == "counters":
        ents = counter_table(a.pmc_dirs, a.trace_dir, a.match, a.copy_mib, a.cus)
        if a.json:
            with open(a.json, "w") as f:
                json.dump(ents, f, indent=1)
        print("\n".join(counter_markdown(ents, a.title, a.command)))
        return 0

    if a.cmd == "stats":
        lines, total = kernel_table(a.dir)
        last = last_dispatches(a.dir, a.kernel, a.reps)
        avg_us = sum(d for _, d in last) / len(last) / 1e3
        print(f"# {a.title}\n\nCommand (repo root, ``cd /tmp && export TMPDIR=/tmp`` first):\n\n"
              f"    {a.command}\n\nAll dispatches of the run (stage steps, warmup and isolated kernel "
              f"launches), total {total / 1e6:.3f} ms of kernel time.\n")
        print("\n".join(lines))
        print(f"\nIsolated launches: last {len(last)} dispatches matching `{a.kernel}`: "
              f"average {avg_us:.2f} us (min {min(d for _, d in last) / 1e3:.2f}, "
              f"max {max(d for _, d in last) / 1e3:.2f}).")
    else:
        r = traffic(a.fetch_dir, a.write_dir, a.kernel, a.reps, a.copy_mib)
        r.update({"kernel": a.kernel, "copy_mib": a.copy_mib,
                  "command_fetch": a.command_fetch, "command_write": a.command_write})
        with open(a.json, "w") as f:
            json.dump(r, f, indent=1)
        rd, wr = r["read"], r["write"]
        print(f"# HBM traffic per launch of `{a.kernel}`\n\nCommands (repo root, ``cd /tmp && export "
              f"TMPDIR=/tmp`` first):\n\n    {a.command_fetch}\n    {a.command_write}\n")
        print("| counter | kernel KiB/dispatch | copy KiB/dispatch | copy true KiB | factor | bytes |")
        print("|---|---:|---:|---:|---:|---:|")
        for x in (rd, wr):
            print(f"| {x['counter']} | {x['kernel_kib']:.0f} (n={x['kernel_dispatches']}) | {x['copy_kib']:.0f} "
                  f"(n={x['copy_dispatches']}) | {a.copy_mib * 1024} | {x['factor']:.4f} | {x['bytes']:.4g} |")
        print(f"\nHBM bytes per launch (read + write): {r['hbm_bytes_per_launch']:.6g}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
