"""Benchmark of orth(X) on one MI355X: microseconds per orth() call, max|Q^T Q - I|, and the roofline of each kernel.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--cpu-seconds S] [--no-cpu] [--no-graph] [--headline-only]

Workload (the quoted target shapes): one orth() call at 768x512 (the 110M attention layer: X = V (U^T U) + u^T U with
N = 768, U's singular values log-uniform over [1, 1e4], u unit-RMS Gaussian, seed 0) and one at 17408x256 (the 27B
down_proj layer, same generator with N = 5120), generated on the CPU and resident on the GPU before timing. Each
input has its own captured hipGraph; one step replays both. `value` = timed wall time / (steps x 2) in microseconds
per call (lower is better); the per-shape figures and their targets are in `targets`, right after `orth_max`.

Per headline shape, as the reference's qrbench/bench.py:28-53 measures: "thr" (median of 5 bursts of 20
back-to-back replays), "lat" (one replay between two events after a synchronisation, median of 20) and "lat_flush"
(the same after overwriting a 512 MiB buffer, which evicts the L2s and the 256 MiB MALL), plus every kernel's average
launch duration (HIP events around back-to-back launches on the call's stream) with its algorithmic flops and bytes
as fractions of the MFMA and HBM peaks, the roofline of the dominant kernel, the Cholesky's per-step critical path
(device wall clock) and the gap between the graph replay and the summed kernel times.

Secondary lines: the 0.8B layer shapes (1024x256, 2048x256, 3584x256, two seeds each), 2048x512, 5120x256 and
6144x256 (the 27B layer shapes with the algorithmic GB/s of each pass's Gram and Cholesky + solve, `pass_gbs`), the
27B layers wider than 512 (block Gram-Schmidt), the batched layer set (12 x 768x512 + 12 x 2048x512,
one hipGraph per shape group, against 24 single-call graphs) and a CPU baseline on a bounded sample at the two
headline shapes (the C restatement in oracle/ with OpenMP on the host, and CPU torch.linalg.qr).

--headline-only runs the timed region alone and prints its line (the command the rocprofv3 summaries in profiles/
come from). --detail PATH also writes every measured figure to PATH as JSON.
"""
import argparse
import ctypes
import json
import os
import statistics
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from spanqr_amd import _lib, kcholqr_f, kcholqr_f_many, orth, stages  # noqa: E402
from spanqr_amd.plan import get_plan, stream_handle  # noqa: E402
from spanqr_amd.qrbench import gen  # noqa: E402

METRIC = "µs per orth() call at K×r (median); max|QᵀQ−I|; % of HBM/MFMA roofline"
# (name, K, r, generator arguments): the two shapes the targets are quoted at
HEADLINE = [("768x512", 768, 512, {"N": 768, "seed": 0}), ("17408x256", 17408, 256, {"N": 5120, "seed": 0})]
TARGET_US = {"768x512": 250.0, "17408x256": 350.0}
WORKLOAD_08B = [(1024, 256), (2048, 256), (3584, 256)]
SEEDS_08B = (0, 1)
OTHER_SHAPES = [(2048, 512), (5120, 256), (6144, 256)]
# 27B layers wider than 512 (orth.py:18-19: block Gram-Schmidt over 256-column blocks, candidates/kbig.py:69-95)
BLOCKED_SHAPES = [(5120, 1024), (17408, 1024), (17408, 2048)]
BATCH_GROUPS = [(768, 512, 12), (2048, 512, 12)]   # the 110M model's attention and down_proj layers
PEAK_FP32_TFLOPS = 157.3     # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
FLUSH_BYTES = 512 << 20      # more than the 256 MiB MALL plus every XCD's L2


# kernel families of one call: (name, spanqr_profile_kernel id, launches per call); a plan whose solve runs in the
# Cholesky's launch has chol_solve families in place of chol and trsm
FAMILIES = [("amax", _lib.K_AMAX, 1), ("gram_pass1", _lib.K_GRAM_PASS1, 1), ("gram", _lib.K_GRAM, 4),
            ("reduce", _lib.K_REDUCE, 5), ("chol", _lib.K_CHOL, 3), ("trsm_pass1", _lib.K_TRSM_PASS1, 1),
            ("trsm", _lib.K_TRSM, 2), ("ns_apply", _lib.K_NS_APPLY, 2)]
FUSED_FAMILIES = [("amax", _lib.K_AMAX, 1), ("gram_pass1", _lib.K_GRAM_PASS1, 1), ("gram", _lib.K_GRAM, 4),
                  ("reduce", _lib.K_REDUCE, 5), ("chol_solve_pass1", _lib.K_CHOL_SOLVE_PASS1, 1),
                  ("chol_solve", _lib.K_CHOL_SOLVE, 2), ("ns_apply", _lib.K_NS_APPLY, 2)]


def algorithmic(family, K, r):
    """(flops, HBM bytes) of one launch at (K, r): Gram K r (r+1) flops (symmetric half) reading X once; solve
    K r (r+1) flops reading A (and Z on pass 1) and writing Y; NS apply 2 K r^2 flops reading Y and writing Q;
    Cholesky r^3 / 3 flops; amax reads X; the reduce moves only r x r partials (not counted)."""
    kr = 4.0 * K * r
    return {"amax": (0.0, kr), "gram_pass1": (K * r * (r + 1.0), kr), "gram": (K * r * (r + 1.0), kr),
            "reduce": (0.0, 0.0), "chol": (r ** 3 / 3.0, 0.0), "trsm_pass1": (K * r * (r + 1.0), 3 * kr),
            "trsm": (K * r * (r + 1.0), 2 * kr), "ns_apply": (2.0 * K * r * r, 2 * kr),
            "chol_solve_pass1": (r ** 3 / 3.0 + K * r * (r + 1.0), 3 * kr),
            "chol_solve": (r ** 3 / 3.0 + K * r * (r + 1.0), 2 * kr)}[family]


def call_work(K, r):
    """(flops, bytes) of one orth() call: 8 K r (r+1) + 4 K r^2 + r^3 flops, 68 K r bytes (17 fp32 passes over X)"""
    return 8.0 * K * r * (r + 1) + 4.0 * K * r * r + float(r) ** 3, 68.0 * K * r


def kernel_avg_us(X, which, reps):
    """average duration of one kernel of the call at X's shape: reps back-to-back launches between two HIP events on
    the current stream (spanqr_profile_kernel), after one orth() call has filled the plan's workspace"""
    K, r = X.shape
    kcholqr_f(X)
    plan = get_plan(K, r, X.device)
    ms = ctypes.c_float()
    _lib.check(_lib.lib().spanqr_profile_kernel(plan.handle, which, reps, ctypes.byref(ms), stream_handle(X.device)))
    return ms.value * 1000.0


def chol_steps_us(X):
    """per 32-column diagonal step of the Cholesky: the device wall clock stamped by workgroup 0 of an instrumented
    copy of the kernel (spanqr_profile_chol), warm (the median of five launches after two untimed ones, per step):
    (list of step us, factorisation us)"""
    K, r = X.shape
    kcholqr_f(X)
    plan = get_plan(K, r, X.device)
    G, npart = stages.gram(X, kahan=True, use_scale=True)
    nb = r // 32
    runs = []
    for rep in range(7):
        stamps = (ctypes.c_ulonglong * (24 * nb + 2))()
        tick = ctypes.c_double()
        _lib.check(_lib.lib().spanqr_profile_chol(plan.handle, G.data_ptr(), npart.data_ptr(), 1e-7, 1e-8, stamps,
                                                  ctypes.byref(tick), stream_handle(X.device)))
        us = lambda a, b: (stamps[b] - stamps[a]) * tick.value / 1000.0
        if rep >= 2:
            runs.append(([us(1 + 4 * j, 1 + 4 * (j + 1)) for j in range(nb)], us(0, 1 + 4 * nb)))
    steps = [round(statistics.median(rn[0][j] for rn in runs), 2) for j in range(nb)]
    return steps, round(statistics.median(rn[1] for rn in runs), 2)


def traffic_bytes(family, shape):
    """HBM bytes per launch of a kernel family at a shape, from the rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs
    recorded in profiles/traffic.json (None if there is no record)"""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            rec = json.load(f).get(shape, {}).get(family)
    except (OSError, ValueError, AttributeError):
        return None
    return None if rec is None else rec.get("bytes_per_launch")


def capture(X, fn=None):
    """(graph, Q): one orth() call on X captured into a hipGraph on a side stream (plan created beforehand)"""
    fn = fn or kcholqr_f
    st = torch.cuda.Stream(X.device)
    st.wait_stream(torch.cuda.current_stream(X.device))
    with torch.cuda.stream(st):
        fn(X)                      # creates the plan for this stream and warms up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        Q = fn(X)
    torch.cuda.synchronize()
    return g, Q


class _Direct:
    """direct launches in place of a graph (--no-graph)"""

    def __init__(self, X, fn=None):
        self.X, self.fn = X, fn or kcholqr_f
        self.Q = self.fn(X)

    def replay(self):
        self.Q = self.fn(self.X)


def runner(X, graphs, fn=None):
    if graphs:
        return capture(X, fn)
    d = _Direct(X, fn)
    return d, d.Q


def capture_many(Xs):
    """(graph, [Q]): one batched call on the same-shape list Xs captured into a hipGraph on a side stream"""
    st = torch.cuda.Stream(Xs[0].device)
    st.wait_stream(torch.cuda.current_stream(Xs[0].device))
    with torch.cuda.stream(st):
        kcholqr_f_many(Xs)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        Qs = kcholqr_f_many(Xs)
    torch.cuda.synchronize()
    return g, Qs


def time_rounds(graphs, steps, reps=5):
    """median over `reps` of the time of `steps` rounds of replaying every graph once, microseconds per round"""
    out = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(steps):
            for g in graphs:
                g.replay()
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e) * 1000.0 / steps)
    return statistics.median(out)


def thr_us(g, n=20, reps=5):
    """back-to-back: median over `reps` bursts of n replays, microseconds per replay (qrbench/bench.py:44-52)"""
    return time_rounds([g], n, reps)


def lat_us(g, n=20, flush=None):
    """isolated call: one replay between two events after a synchronisation, median of n (qrbench/bench.py:36-43);
    with `flush` (a device buffer) overwritten before each sample so that no cache holds the inputs"""
    out = []
    for _ in range(n):
        if flush is not None:
            flush.zero_()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        g.replay()
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e) * 1000.0)
    return statistics.median(out)


def orth_error(Q):
    Qd = Q.detach().double().cpu()
    return float((Qd.T @ Qd - torch.eye(Q.shape[1], dtype=torch.float64)).abs().max())


def kernels_at(X, reps):
    """per kernel family at X's shape: average launch duration and its algorithmic rates"""
    K, r = X.shape
    kcholqr_f(X)
    plan = get_plan(K, r, X.device)
    fams = FUSED_FAMILIES if plan.solve_rows > 0 else FAMILIES
    if plan.gram_short:   # the Gram reduces its splits in its own launch
        fams = [f for f in fams if f[0] != "reduce"]
    out = {}
    for fam, which, per_call in fams:
        us = kernel_avg_us(X, which, reps)
        fl, by = algorithmic(fam, K, r)
        out[fam] = {"us": round(us, 3), "per_call": per_call, "tflops": round(fl / us / 1e6, 3),
                    "gbs": round(by / us / 1e3, 1), "mfma_frac": round(fl / us / 1e6 / PEAK_FP32_TFLOPS, 5),
                    "hbm_frac": round(by / us / 1e3 / PEAK_HBM_GBS, 5)}
    return out


def roofline_of(kern, shapes):
    """roofline of the kernel family with the largest share of the summed kernel time over the headline shapes:
    achieved = mean algorithmic work per launch / mean launch duration (both over one launch at each shape, as a
    trace of the timed region averages them)"""
    tot = {fam: sum(kern[s][fam]["us"] * kern[s][fam]["per_call"] for s in shapes if fam in kern[s])
           for fam in kern[shapes[0]]}
    dom = max(tot, key=tot.get)
    dims = {name: (K, r) for name, K, r, _ in HEADLINE}
    fl = statistics.mean(algorithmic(dom, *dims[s])[0] for s in shapes)
    by = statistics.mean(algorithmic(dom, *dims[s])[1] for s in shapes)
    shapes = [s for s in shapes if dom in kern[s]]
    us = statistics.mean(kern[s][dom]["us"] for s in shapes)
    bound = "mfma" if fl / PEAK_FP32_TFLOPS >= by / PEAK_HBM_GBS * 1e-3 else "hbm"
    achieved = fl / us / 1e6 if bound == "mfma" else by / us / 1e3
    peak = PEAK_FP32_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
    traffic = [traffic_bytes(dom, s) for s in shapes]
    return {"bound": bound, "achieved": achieved, "peak": peak, "unit": "TFLOP/s" if bound == "mfma" else "GB/s",
            "frac": achieved / peak, "traffic": statistics.mean(traffic) if None not in traffic else None,
            "kernel": dom, "avg_launch_us": us, "work_per_launch": fl if bound == "mfma" else by,
            "share_of_kernel_time": tot[dom] / sum(tot.values())}


def cpu_baseline(inputs, seconds):
    """the oracle (C restatement, OpenMP) and CPU torch.linalg.qr on the host, on a bounded sample"""
    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    per_shape, hh = {}, {}
    budget = seconds / max(1, len(inputs))
    for name, X in inputs.items():
        K, r = X.shape
        Xn = X.cpu().numpy()
        KS = get_plan(K, r, X.device).split_rows
        oracle.orth(Xn, KS)                                  # warm-up
        times, t_end = [], time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            oracle.orth(Xn, KS)
            times.append(time.perf_counter() - t0)
        per_shape[name] = round(statistics.median(times) * 1e6, 1)
        Xc = X.cpu()
        torch.linalg.qr(Xc)
        ht = []
        for _ in range(5):
            t0 = time.perf_counter()
            torch.linalg.qr(Xc)
            ht.append(time.perf_counter() - t0)
        hh[name] = round(statistics.median(ht) * 1e6, 1)
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": statistics.mean(per_shape.values()), "unit": "us/call", "cores": threads, "kind": "port",
        "sample": f"oracle/kcholf_oracle.c orth() of the headline inputs ({', '.join(inputs)}), median over "
                  f">= {budget:.1f} s each (OpenMP, {threads} threads)",
        "per_shape_us": per_shape, "torch_linalg_qr_us": hh, "cpu_model": model, "cpu_count": os.cpu_count(),
    }


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-graph", action="store_true", help="direct launches instead of one hipGraph per input")
    p.add_argument("--kernel-reps", type=int, default=100, help="launches per kernel timing")
    p.add_argument("--headline-only", action="store_true", help="only the timed region (for profiling runs)")
    p.add_argument("--detail", default=None, help="also write every figure to this JSON file")
    a = p.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py measures one GPU: orth() of one matrix runs on a single MI355X and this build has no "
              f"multi-GPU path, so --gpus {a.gpus} is not supported", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    graphs = not a.no_graph

    inputs = {name: gen.ttf_uu(K, r, **kw).to(dev) for name, K, r, kw in HEADLINE}
    runs = {name: runner(X, graphs) for name, X in inputs.items()}
    for _ in range(a.warmup):
        for g, _q in runs.values():
            g.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(a.steps):
        for g, _q in runs.values():
            g.replay()
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    value = total_ms * 1000.0 / (a.steps * len(runs))
    orth_max = max(orth_error(q) for _g, q in runs.values())
    line = {
        "metric": METRIC, "value": value, "unit": "us/call", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": total_ms / a.steps, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "orth() at 768x512 (110M attention layer, N=768) and 17408x256 (27B down_proj "
                               "layer, N=5120), cond(U^T U) ~1e8 generator, seed 0, one hipGraph per input, both "
                               "per step", "shapes": list(runs), "calls_per_step": len(runs), "graphs": graphs},
        "orth_max": orth_max,
    }
    if a.headline_only:
        print(json.dumps(line), flush=True)
        return 0

    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    head, kern = {}, {}
    for name, K, r, _kw in HEADLINE:
        g, q = runs[name]
        ks = kernels_at(inputs[name], a.kernel_reps)
        kern[name] = ks
        t = thr_us(g)
        summed = sum(v["us"] * v["per_call"] for v in ks.values())
        F, B = call_work(K, r)
        steps, chol_us = chol_steps_us(inputs[name])
        head[name] = {"thr_us": round(t, 2), "lat_us": round(lat_us(g), 2), "lat_flush_us": round(lat_us(g, flush=flush), 2),
                      "orth": orth_error(q), "sum_of_kernels_us": round(summed, 2), "gap_us": round(t - summed, 2),
                      "call_mfma_frac": round(F / (t * 1e-6) / 1e12 / PEAK_FP32_TFLOPS, 4),
                      "call_hbm_frac": round(B / (t * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
                      "chol_us": chol_us, "chol_step_us": steps,
                      "kernels_us": {fam: v["us"] for fam, v in ks.items()}}
    del flush
    roofline = roofline_of(kern, list(head))

    w08 = {}
    for K, r in WORKLOAD_08B:
        ts = []
        for s in SEEDS_08B:
            g, _q = runner(gen.ttf_uu(K, r, N=K, seed=s).to(dev), graphs)
            ts.append(thr_us(g))
        w08[f"{K}x{r}"] = round(statistics.mean(ts), 2)
    others = {}
    for K, r in OTHER_SHAPES:
        X = gen.bench_input(K, r, seed=0).to(dev)
        g, q = runner(X, graphs)
        others[f"{K}x{r}"] = {"thr_us": round(thr_us(g), 2), "lat_us": round(lat_us(g), 2), "orth": orth_error(q)}
        if r == 256:
            # the 27B layer shapes: the algorithmic GB/s of each pass's Gram (SYRK) and Cholesky + solve (TRSM)
            ks = kernels_at(X, a.kernel_reps)
            kern[f"{K}x{r}"] = ks
            others[f"{K}x{r}"]["pass_gbs"] = {fam: v["gbs"] for fam, v in ks.items()}
        del g, q, X
    blocked = {}
    for K, r in BLOCKED_SHAPES:
        X = gen.bench_input(K, r, seed=0).to(dev)
        g, q = runner(X, graphs, orth)
        blocked[f"{K}x{r}"] = {"thr_us": round(thr_us(g, n=5), 1), "lat_us": round(lat_us(g, n=5), 1),
                               "orth": orth_error(q), "blocks": r // 256}
        del g, q, X
    torch.cuda.synchronize()
    batched = batched_layers(dev, max(1, min(a.steps, 20)))

    cpu = None if a.no_cpu else cpu_baseline(inputs, a.cpu_seconds)
    targets = {name: {"us_per_call": head[name]["thr_us"], "target_us": TARGET_US[name],
                      "met": head[name]["thr_us"] <= TARGET_US[name], "lat_us": head[name]["lat_us"],
                      "orth": head[name]["orth"], "chol_us": head[name]["chol_us"]} for name in head}
    # the per-shape targets right after the headline fields, so that a reader of the line's first part sees them
    line.update({
        "targets": targets, "roofline": roofline, "cpu_baseline": cpu, "headline": head,
        "shapes_0.8b_thr_us": w08, "shapes": others, "blocked_shapes": blocked, "batched_layers": batched,
        "device": torch.cuda.get_device_name(dev),
    })
    if a.detail:
        with open(a.detail, "w") as f:
            json.dump({"line": line, "kernels": kern}, f, indent=1)
    print(json.dumps(line), flush=True)
    return 0


def batched_layers(dev, steps):
    """the batched layer set: per training step, orth of 12 layers at 768x512 and 12 at 2048x512 (independent
    inputs of the cond-1e8 generator, seeds 100 + 12 g + i), as two batched graphs (one per shape group) and as 24
    single-call graphs; Q of the two forms compared bit for bit"""
    groups = []
    for gi, (K, r, n) in enumerate(BATCH_GROUPS):
        groups.append([gen.ttf_uu(K, r, N=K, seed=100 + 12 * gi + i).to(dev) for i in range(n)])
    single = [capture(X) for grp in groups for X in grp]
    batched = [capture_many(grp) for grp in groups]
    for g, _q in single + batched:
        g.replay()
    torch.cuda.synchronize()
    q_single = [q for _g, q in single]
    q_batched = [q for _g, qs in batched for q in qs]
    same = all(torch.equal(a.view(torch.int32), b.view(torch.int32)) for a, b in zip(q_single, q_batched))
    t_single = time_rounds([g for g, _q in single], steps)
    t_batched = time_rounds([g for g, _q in batched], steps)
    res = {"groups": [f"{n} x {K}x{r}" for K, r, n in BATCH_GROUPS],
           "us_per_step_batched": round(t_batched, 1), "us_per_step_sequential": round(t_single, 1),
           "speedup": round(t_single / t_batched, 2), "bitwise_equal_to_single_calls": same,
           "orth_max": max(orth_error(q) for q in q_batched)}
    del single, batched
    torch.cuda.synchronize()
    return res


if __name__ == "__main__":
    sys.exit(main())
