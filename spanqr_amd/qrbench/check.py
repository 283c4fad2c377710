"""Accuracy and robustness check of orth(X) on the GPU, case by case, against the requirements in metrics.py.

    python -m spanqr_amd.qrbench.check                                    # acceptance + extra cases, bench shapes
    python -m spanqr_amd.qrbench.check --shapes 768x512 --cases mixed ttf --target
    python -m spanqr_amd.qrbench.check --real dumps/ --real-only          # matrices dumped from a training run

For every matrix the fp64 reference is built once; every method named with -m (orth: this library; householder:
torch.linalg.qr) is run through metrics.check_call, and Householder's span error on the same matrix sets the span
bar. --target uses this project's 2e-7 orthogonality bar instead of the reference's 1e-6. Exit status 0 when every
acceptance ("hard") case of every method passes. The cases and the requirements are the reference's (qrbench/gen.py,
qrbench/metrics.py); this command line is this project's own.
"""
import argparse
import json
import sys
import time
from dataclasses import asdict, dataclass, field

import torch

from . import gen, metrics


def _orth():
    from spanqr_amd import orth     # the native path; raises if the library is missing
    return orth


METHODS = {"orth": _orth, "householder": lambda: metrics.householder}


def parse_shapes(spec):
    """shape list from: bench | all | a model name (110m, 0.8b, 27b) | KxR[,KxR...]"""
    named = {"bench": gen.BENCH_SHAPES, "all": gen.ALL_SHAPES, **gen.SHAPES}
    if spec in named:
        return list(named[spec])
    return [tuple(int(v) for v in item.split("x")) for item in spec.split(",")]


@dataclass
class Record:
    """one (method, matrix) outcome"""
    method: str
    K: int
    r: int
    case: str
    hard: bool
    cond: float
    hh_span_n: float
    fails: list = field(default_factory=list)
    report: dict = field(default_factory=dict)

    def line(self):
        tag = "ok  " if not self.fails else ("FAIL" if self.hard else "fail")
        rep = self.report
        return (f"{tag} {self.method:<12} {self.K:>5}x{self.r:<4} {self.case:<28} cond {self.cond:8.1e} "
                f"orth {rep.get('orth', float('nan')):8.1e} span_n {rep.get('span_n', 0.0):7.3g} "
                f"(hh {self.hh_span_n:6.3g})  {'; '.join(self.fails)}")


def cases_for(K, r, names, seeds, real, extra):
    """the synthetic cases (none when names == []) and, with real, the dumped matrices of this shape"""
    if names != []:
        yield from gen.make_cases(K, r, names, seeds, include_extra=extra)
    if real:
        yield from gen.real_cases(real, (K, r))


def check_case(case, fns, device, orth_tol, check_sync):
    """Records of every method on one case"""
    K, r = case.X.shape
    X = case.X.to(device)
    ref = metrics.reference(case.X)
    hh, _ = metrics.check_call(metrics.householder, X, ref, check_sync=False)
    out = []
    for name, fn in fns.items():
        rep, _ = metrics.check_call(fn, X, ref, check_sync=check_sync)
        out.append(Record(name, K, r, case.name, case.hard, ref.cond, hh.span_n,
                          rep.failures(span_ref=hh.span_n, orth_tol=orth_tol), rep.as_dict()))
    return out


def tally(records):
    """per method: passed/total acceptance cases, passed/total extra cases, worst orth, failing acceptance cases"""
    out = {}
    for rec in records:
        t = out.setdefault(rec.method, {"hard": [0, 0], "extra": [0, 0], "worst_orth": 0.0, "hard_failures": []})
        kind = t["hard"] if rec.hard else t["extra"]
        kind[0] += not rec.fails
        kind[1] += 1
        orth = rec.report.get("orth", float("nan"))
        if orth == orth:
            t["worst_orth"] = max(t["worst_orth"], orth)
        if rec.hard and rec.fails:
            t["hard_failures"].append(f"{rec.K}x{rec.r} {rec.case}: {'; '.join(rec.fails)}")
    return out


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("-m", "--methods", nargs="+", default=["orth"], choices=sorted(METHODS))
    p.add_argument("--shapes", default="bench", help="bench | all | 110m | 0.8b | 27b | KxR[,KxR...]")
    p.add_argument("--cases", nargs="*", help="case names or prefixes (default: all)")
    p.add_argument("--seeds", type=int, default=1)
    p.add_argument("--real", help="directory of dumped X matrices (spanqr_amd.qrbench.dump or the reference's)")
    p.add_argument("--real-only", action="store_true", help="only the dumped matrices (with --real)")
    p.add_argument("--no-extra", action="store_true", help="acceptance cases only")
    p.add_argument("--no-sync-check", action="store_true")
    p.add_argument("--target", action="store_true", help="orthogonality bar 2e-7 instead of the reference's 1e-6")
    p.add_argument("--json", help="write every record to this file")
    a = p.parse_args(argv)
    t0 = time.time()
    fns = {name: METHODS[name]() for name in a.methods}
    tol = metrics.ORTH_TOL_TARGET if a.target else metrics.ORTH_TOL
    names = [] if a.real_only else a.cases
    records = []
    for K, r in parse_shapes(a.shapes):
        for case in cases_for(K, r, names, tuple(range(a.seeds)), a.real, not a.no_extra):
            for rec in check_case(case, fns, "cuda", tol, not a.no_sync_check):
                records.append(rec)
                print(rec.line(), flush=True)
    summary = tally(records)
    for name, t in summary.items():
        print(f"{name}: acceptance {t['hard'][0]}/{t['hard'][1]}, extra {t['extra'][0]}/{t['extra'][1]}, "
              f"worst orth {t['worst_orth']:.2e}")
        for f in t["hard_failures"]:
            print(f"    FAIL {f}")
    print(f"({time.time() - t0:.0f} s, {torch.cuda.get_device_name()})")
    if a.json:
        with open(a.json, "w") as fh:
            json.dump({"device": torch.cuda.get_device_name(), "records": [asdict(r) for r in records],
                       "summary": summary}, fh, indent=1)
    return 0 if all(t["hard"][0] == t["hard"][1] for t in summary.values()) else 1


if __name__ == "__main__":
    sys.exit(main())
