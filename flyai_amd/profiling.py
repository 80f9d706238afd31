"""Summaries of rocprofv3 CSV output (``-f csv``) for the stage step and the MXFP4 expert kernels.

Two reports, both plain text for committing beside the numbers they support:

* ``stats``: the ``--kernel-trace --stats`` kernel table of a ``bench.py`` run, plus the average
  duration of the last ``reps`` dispatches of one kernel (the isolated launches ``bench.py`` times
  with HIP events after the stage steps);
* ``traffic``: HBM bytes per launch of one kernel from two ``--pmc`` runs (``FETCH_SIZE`` and
  ``WRITE_SIZE``, KiB per dispatch).  Each reading is scaled by the reading of a plain device copy
  of known size in the same run (``bench.py --copy-probe-mib M``): factor = M MiB / copy reading.

Usage (after the rocprofv3 runs, on any machine)::

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
    a = ap.parse_args(argv)

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
