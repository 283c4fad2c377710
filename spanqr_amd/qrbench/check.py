"""Accuracy / robustness check of orth(X) on the MI355X against the reference's requirements (qrbench/check.py).

    python -m spanqr_amd.qrbench.check                                   # all cases, acceptance shapes
    python -m spanqr_amd.qrbench.check --shapes 768x512 --cases mixed ttf
    python -m spanqr_amd.qrbench.check --real dumps/ --real-only          # matrices dumped from training

Every case also runs through Householder QR (torch.linalg.qr, the span reference: orth must be within SPAN_RATIO of
it). Per case: run_checked (warm-up, a call under torch's sync-debug "error" mode, a determinism call, input left
intact) and the hard requirements of qrbench/metrics.py; --target also applies this build's tighter orthogonality
gate (2e-7). The exit status is 0 when every acceptance case passes.
"""
import argparse
import json
import sys
import time

import torch

from . import gen, metrics

METHODS = {"orth": None, "householder": metrics.householder}


def _method(name):
    if name == "orth":
        from spanqr_amd import orth     # the native path; raises if the library is missing
        return orth
    return METHODS[name]


def parse_shapes(spec):
    """bench | all | 110m | 0.8b | 27b | KxR[,KxR...] (qrbench/check.py:19-26)"""
    if spec == "bench":
        return gen.BENCH_SHAPES
    if spec == "all":
        return gen.ALL_SHAPES
    if spec in gen.SHAPES:
        return gen.SHAPES[spec]
    return [tuple(int(v) for v in s.split("x")) for s in spec.split(",")]


def run(method_names, shapes, case_names=None, seeds=(0,), real=None, extra=True, check_sync=True, target=False,
        device="cuda", verbose=True):
    """rows of results, one per (method, shape, case) -- qrbench/check.py:29-48"""
    fns = {n: _method(n) for n in method_names}
    rows = []
    for K, r in shapes:
        cases = [] if case_names == ["__none__"] else list(gen.make_cases(K, r, case_names, seeds, include_extra=extra))
        if real:
            cases += list(gen.real_cases(real, (K, r)))
        for case in cases:
            X = case.X.to(device)
            ref = metrics.reference(case.X)
            hres, _ = metrics.run_checked(metrics.householder, X, ref, check_sync=False)
            cond = float(ref[0][0] / ref[0][-1]) if ref[0][-1] > 0 else float("inf")
            for n, fn in fns.items():
                res, _ = metrics.run_checked(fn, X, ref, check_sync=check_sync)
                tol = metrics.ORTH_TOL_TARGET if target else metrics.ORTH_TOL
                fails = res.failures(span_ref=hres.span_n, orth_tol=tol)
                row = dict(method=n, K=K, r=r, case=case.name, hard=case.hard, cond=cond, hh_span_n=hres.span_n,
                           fails=fails, **res.as_dict())
                rows.append(row)
                if verbose:
                    _print_row(row)
    return rows


def _fmt(v, f="{:.1e}"):
    return "-" if v is None or v != v else f.format(v)


def _print_row(w):
    status = "ok  " if not w["fails"] else ("FAIL" if w["hard"] else "fail")
    print(f"{status} {w['method']:<12} {w['K']:>5}x{w['r']:<4} {w['case']:<28} cond {_fmt(w['cond'], '{:.0e}'):>6}"
          f"  orth {_fmt(w['orth']):>7}  span_n {_fmt(w['span_n'], '{:.3g}'):>7} (hh {_fmt(w['hh_span_n'], '{:.3g}'):>6})"
          f"  {'; '.join(w['fails'])}", flush=True)


def summarize(rows):
    print("\nsummary (hard = acceptance cases, extra = robustness cases):")
    for n in dict.fromkeys(w["method"] for w in rows):
        mine = [w for w in rows if w["method"] == n]
        hard = [w for w in mine if w["hard"]]
        extra = [w for w in mine if not w["hard"]]
        worst = max((w["orth"] for w in mine if w["orth"] == w["orth"]), default=float("nan"))
        print(f"  {n:<12} hard {sum(not w['fails'] for w in hard)}/{len(hard)}  "
              f"extra {sum(not w['fails'] for w in extra)}/{len(extra)}  worst orth {_fmt(worst)}")
        for w in hard:
            if w["fails"]:
                print(f"      FAIL {w['K']}x{w['r']} {w['case']}: {'; '.join(w['fails'])}")


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
    p.add_argument("--target", action="store_true", help="orthogonality gate 2e-7 instead of the reference's 1e-6")
    p.add_argument("--json", help="write all rows to this file")
    a = p.parse_args(argv)
    t0 = time.time()
    cases = ["__none__"] if a.real_only else a.cases
    rows = run(a.methods, parse_shapes(a.shapes), cases, tuple(range(a.seeds)), a.real, extra=not a.no_extra,
               check_sync=not a.no_sync_check, target=a.target)
    summarize(rows)
    print(f"({time.time() - t0:.0f} s, {torch.cuda.get_device_name()})")
    if a.json:
        with open(a.json, "w") as f:
            json.dump(dict(device=torch.cuda.get_device_name(), rows=rows), f, indent=1)
    return 0 if all(not w["fails"] for w in rows if w["hard"]) else 1


if __name__ == "__main__":
    sys.exit(main())
