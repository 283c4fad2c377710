"""Summaries of rocprofv3 CSV output for orth().

    python3 -m spanqr_amd.qrbench.rocprof_summary trace KERNEL_TRACE.csv
        per kernel and grid: dispatches, average / median / min / max duration (us) and share of the total
    python3 -m spanqr_amd.qrbench.rocprof_summary traffic FETCH.csv WRITE.csv [--json OUT]
        HBM bytes per launch of each kernel of the call (counter runs of spanqr_amd.qrbench.traffic): FETCH_SIZE and
        WRITE_SIZE per dispatch (KiB), each scaled by the ratio of true to counted bytes of a plain 512 MiB copy
"""
import argparse
import csv
import json
import re
import statistics
import sys

OURS = ("k_amax", "k_gram", "k_reduce", "k_chol", "k_trsm", "k_nsapply")


def short_name(name):
    n = re.sub(r"\(anonymous namespace\)::", "", name)
    n = re.sub(r"^void ", "", n)
    base = n.split("(")[0]
    return base if len(base) < 60 else base[:57] + "..."


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def trace(path):
    groups = {}
    for r in _rows(path):
        wg = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
        grid = (int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])) // max(wg, 1)
        key = (short_name(r["Kernel_Name"]), grid, wg)
        groups.setdefault(key, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    total = sum(sum(v) for v in groups.values())
    out = ["| kernel | workgroups x size | dispatches | avg us | median us | min us | max us | share |",
           "|---|---|---|---|---|---|---|---|"]
    for (name, grid, wg), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"| {name} | {grid} x {wg} | {len(v)} | {statistics.mean(v):.2f} | {statistics.median(v):.2f} | "
                   f"{min(v):.2f} | {max(v):.2f} | {100 * sum(v) / total:.1f}% |")
    return "\n".join(out)


def _call_families(ns=2):
    fam = ["amax"]
    for p in range(3):
        fam += ["gram_pass1" if p == 0 else "gram", "reduce", "chol", "trsm_pass1" if p == 0 else "trsm"]
    for _ in range(ns):
        fam += ["gram", "reduce", "ns_apply"]
    return fam


def _counter(path, counter):
    """(copy KiB, per-call lists of (family, KiB)) from one counter run of spanqr_amd.qrbench.traffic"""
    rows = [r for r in _rows(path) if r.get("Counter_Name", counter) == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    copy = [float(r["Counter_Value"]) for r in rows if "MulFunctor" in r["Kernel_Name"]]
    ours = [(short_name(r["Kernel_Name"]), float(r["Counter_Value"])) for r in rows
            if any(k in r["Kernel_Name"] for k in OURS)]
    fams = _call_families()
    calls, cur = [], None
    for name, v in ours:
        if name.startswith("k_amax"):
            cur = []
            calls.append(cur)
        if cur is not None:
            cur.append(v)
    calls = [c for c in calls if len(c) == len(fams)]
    return (max(copy) if copy else None), [list(zip(fams, c)) for c in calls]


def traffic(fetch_csv, write_csv, copy_bytes=4 << 27):
    out = {}
    for kind, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE")):
        copy_kib, calls = _counter(path, counter)
        factor = copy_bytes / (copy_kib * 1024.0) if copy_kib else 1.0
        warm = calls[1::2]                      # the driver calls orth twice per shape: keep the second call
        per = {}
        for call in warm:
            for fam, kib in call:
                per.setdefault(fam, []).append(kib * 1024.0 * factor)
        for fam, v in per.items():
            out.setdefault(fam, {})[f"{kind}_bytes_per_launch"] = statistics.mean(v)
        out.setdefault("_scale", {})[f"{kind}_factor"] = factor
    for fam, d in out.items():
        if fam != "_scale":
            d["bytes_per_launch"] = d.get("fetch_bytes_per_launch", 0.0) + d.get("write_bytes_per_launch", 0.0)
    return out


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = p.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    f = sub.add_parser("traffic")
    f.add_argument("fetch_csv")
    f.add_argument("write_csv")
    f.add_argument("--json")
    a = p.parse_args(argv)
    if a.cmd == "trace":
        print(trace(a.csv))
        return 0
    res = traffic(a.fetch_csv, a.write_csv)
    print("| kernel | fetch bytes/launch | write bytes/launch | total |")
    print("|---|---|---|---|")
    for fam, d in res.items():
        if fam == "_scale":
            continue
        print(f"| {fam} | {d.get('fetch_bytes_per_launch', 0):.0f} | {d.get('write_bytes_per_launch', 0):.0f} | "
              f"{d['bytes_per_launch']:.0f} |")
    print(f"\nscale factors (true / counted bytes of a 512 MiB copy): {res['_scale']}")
    if a.json:
        with open(a.json, "w") as fh:
            json.dump(res, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
