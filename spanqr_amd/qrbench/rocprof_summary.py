"""Summaries of rocprofv3 CSV output for orth().

    python3 -m spanqr_amd.qrbench.rocprof_summary trace KERNEL_TRACE.csv
        per kernel and grid: dispatches, average / median / min / max duration (us) and share of the total
    python3 -m spanqr_amd.qrbench.rocprof_summary traffic FETCH.csv WRITE.csv [--json OUT]
        HBM bytes per launch of each kernel of the call at each target shape (counter runs of
        spanqr_amd.qrbench.traffic): FETCH_SIZE and WRITE_SIZE per dispatch (KiB), each scaled by the ratio of true
        to counted bytes of a plain 512 MiB copy
    python3 -m spanqr_amd.qrbench.rocprof_summary mfma PMC.csv KERNEL_TRACE.csv [--json OUT]
        MFMA instructions per launch (SQ_INSTS_MFMA) and the MFMA pipes' busy fraction over the traced duration
"""
import argparse
import csv
import json
import re
import statistics
import sys

OURS = ("k_amax", "k_gram", "k_reduce", "k_chol", "k_trsm", "k_nsapply", "k_copy_out")


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


def call_families(n_kernels, ns=2):
    """kernel families of one orth() call in launch order, from its number of launches: the solve in the Cholesky's
    launch (chol_solve*) or separate (chol, trsm*), with or without a reduce launch after each Gram"""
    for fused in (True, False):
        for reduce in (True, False):
            fam = ["amax"]
            for p in range(3):
                fam += ["gram_pass1" if p == 0 else "gram"] + (["reduce"] if reduce else [])
                fam += (["chol_solve_pass1" if p == 0 else "chol_solve"] if fused else
                        ["chol", "trsm_pass1" if p == 0 else "trsm"])
            for _ in range(ns):
                fam += ["gram"] + (["reduce"] if reduce else []) + ["ns_apply"]
            if len(fam) == n_kernels:
                return fam
    raise ValueError(f"no call structure has {n_kernels} launches")


def _calls(path, counter):
    """(copy value, [call: [(family, value)]]) from one counter run of spanqr_amd.qrbench.traffic: the dispatches of
    this library grouped into calls, each starting at k_amax"""
    rows = [r for r in _rows(path) if r.get("Counter_Name", counter) == counter]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    copy = [float(r["Counter_Value"]) for r in rows if "MulFunctor" in r["Kernel_Name"]]
    calls = []
    for r in rows:
        if not any(k in r["Kernel_Name"] for k in OURS):
            continue
        if short_name(r["Kernel_Name"]).startswith("k_amax"):
            calls.append([])
        if calls:
            calls[-1].append(float(r["Counter_Value"]))
    return (max(copy) if copy else None), [list(zip(call_families(len(c)), c)) for c in calls]


def traffic(fetch_csv, write_csv, shapes, copy_bytes=4 << 27):
    """per shape and kernel family: HBM bytes per launch from FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled
    by true / counted bytes of the plain copy; the warm (second) call of each shape"""
    out = {"_scale": {}}
    for kind, path, counter in (("fetch", fetch_csv, "FETCH_SIZE"), ("write", write_csv, "WRITE_SIZE")):
        copy_kib, calls = _calls(path, counter)
        factor = copy_bytes / (copy_kib * 1024.0) if copy_kib else 1.0
        out["_scale"][f"{kind}_factor"] = factor
        for shape, call in zip(shapes, calls[1::2]):
            per = {}
            for fam, kib in call:
                per.setdefault(fam, []).append(kib * 1024.0 * factor)
            for fam, v in per.items():
                out.setdefault(shape, {}).setdefault(fam, {})[f"{kind}_bytes_per_launch"] = statistics.mean(v)
    for shape, d in out.items():
        if shape == "_scale":
            continue
        for fam, rec in d.items():
            rec["bytes_per_launch"] = rec.get("fetch_bytes_per_launch", 0.0) + rec.get("write_bytes_per_launch", 0.0)
    return out


def mfma(csv_path, trace_csv, shapes, simds=1024, clock_ghz=2.4):
    """per shape and family: SQ_INSTS_MFMA per launch and the MFMA pipes' busy fraction over the kernel's duration
    (from a kernel trace of the same program): SQ_VALU_MFMA_BUSY_CYCLES (matrix-pipe cycles summed over the SIMDs:
    32 per fp32 16x16x4 MFMA, 64 per fp32 32x32x2) / (SIMDs x duration cycles)"""
    counts = {}
    for counter in ("SQ_INSTS_MFMA", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CYCLES"):
        _, calls = _calls(csv_path, counter)
        for shape, call in zip(shapes, calls[1::2]):
            for fam, v in call:
                counts.setdefault(shape, {}).setdefault(fam, {}).setdefault(counter, []).append(v)
    durs = {}
    rows = [r for r in _rows(trace_csv) if any(k in r["Kernel_Name"] for k in OURS)]
    rows.sort(key=lambda r: int(r.get("Dispatch_Id", 0)))
    calls, cur = [], None
    for r in rows:
        if short_name(r["Kernel_Name"]).startswith("k_amax"):
            cur = []
            calls.append(cur)
        if cur is not None:
            cur.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0)
    for shape, call in zip(shapes, calls[1::2]):
        for fam, us in zip(call_families(len(call)), call):
            durs.setdefault(shape, {}).setdefault(fam, []).append(us)
    out = {}
    for shape, d in counts.items():
        for fam, c in d.items():
            n = statistics.mean(c.get("SQ_INSTS_MFMA", [0.0]))
            busy = statistics.mean(c.get("SQ_VALU_MFMA_BUSY_CYCLES", [0.0]))
            us = statistics.mean(durs.get(shape, {}).get(fam, [float("nan")]))
            out.setdefault(shape, {})[fam] = {
                "mfma_per_launch": n, "us": us,
                "mfma_busy_frac": busy / (simds * us * 1e-6 * clock_ghz * 1e9) if us == us else None,
                "valu_mfma_busy_cycles": busy,
                "sq_busy_cycles": statistics.mean(c.get("SQ_BUSY_CYCLES", [0.0]))}
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
    m = sub.add_parser("mfma")
    m.add_argument("pmc_csv")
    m.add_argument("trace_csv")
    m.add_argument("--json")
    a = p.parse_args(argv)
    from .traffic import SHAPES
    shapes = [name for name, *_ in SHAPES]
    if a.cmd == "trace":
        print(trace(a.csv))
        return 0
    if a.cmd == "mfma":
        res = mfma(a.pmc_csv, a.trace_csv, shapes)
        print("| shape | kernel | MFMAs per launch | launch us (trace) | MFMA busy |")
        print("|---|---|---|---|---|")
        for shape, d in res.items():
            for fam, v in d.items():
                frac = "-" if v["mfma_busy_frac"] is None else f"{100 * v['mfma_busy_frac']:.1f}%"
                print(f"| {shape} | {fam} | {v['mfma_per_launch']:.0f} | {v['us']:.2f} | {frac} |")
        if a.json:
            with open(a.json, "w") as fh:
                json.dump(res, fh, indent=1)
        return 0
    res = traffic(a.fetch_csv, a.write_csv, shapes)
    print("| shape | kernel | fetch bytes/launch | write bytes/launch | total |")
    print("|---|---|---|---|---|")
    for shape, d in res.items():
        if shape == "_scale":
            continue
        for fam, rec in d.items():
            print(f"| {shape} | {fam} | {rec.get('fetch_bytes_per_launch', 0):.0f} | "
                  f"{rec.get('write_bytes_per_launch', 0):.0f} | {rec['bytes_per_launch']:.0f} |")
    print(f"\nscale factors (true / counted bytes of a 512 MiB copy): {res['_scale']}")
    if a.json:
        with open(a.json, "w") as fh:
            json.dump(res, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
