"""Benchmark of orth(X) on one MI355X: microseconds per orth() call, max|Q^T Q - I|, and the roofline of each kernel.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--cpu-seconds S] [--no-cpu] [--no-graph]

Workload (the reference's 0.8B TTF layer shapes): K x r in {1024x256, 2048x256, 3584x256}, two seeds each, X = V (U^T U)
+ u^T U with N = K (U's singular values log-uniform over [1, 1e4], u unit-RMS Gaussian), generated on the CPU and
resident on the GPU before timing. One step = one orth() call on each of the six inputs; every input has its own
captured hipGraph. `value` = timed wall time / (steps x 6) in microseconds (lower is better).

Also reported: per shape, back-to-back ("thr", 20 replays) and isolated synchronised ("lat") time per call, at the
workload shapes and at 768x512, 2048x512, 5120x256, 6144x256 and 17408x256 (768x512 and 17408x256 are the quoted
targets); the 27B layers wider than 512 (5120x1024, 17408x1024, 17408x2048: block Gram-Schmidt over 256-column
blocks); the batched layer set (12 x 768x512 + 12 x 2048x512, one hipGraph per shape group, against 24
single-call graphs); per kernel and shape the average launch duration (HIP events around back-to-back launches on
the call's stream) with its algorithmic flops and bytes, as TFLOP/s and GB/s and as fractions of the MFMA and HBM
peaks; the roofline of the dominant kernel and of the whole call; the Cholesky's latency
per diagonal step; a CPU baseline on a bounded sample (the C restatement in oracle/, OpenMP, on the host, plus CPU
torch.linalg.qr).
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

from spanqr_amd import _lib, kchol, kcholqr_f, kcholqr_f_many, orth, stages  # noqa: E402
from spanqr_amd.plan import get_plan, stream_handle  # noqa: E402
from spanqr_amd.qrbench import gen  # noqa: E402

METRIC = "µs per orth() call at K×r (median); max|QᵀQ−I|; % of HBM/MFMA roofline"
WORKLOAD_SHAPES = [(1024, 256), (2048, 256), (3584, 256)]
SEEDS = (0, 1)
TARGET_SHAPES = [(768, 512), (17408, 256)]
TARGET_US = {"768x512": 250.0, "17408x256": 350.0}
OTHER_SHAPES = [(768, 512), (2048, 512), (5120, 256), (6144, 256), (17408, 256)]
# 27B layers wider than 512 (orth.py:18-19: block Gram-Schmidt over 256-column blocks, candidates/kbig.py:69-95)
BLOCKED_SHAPES = [(5120, 1024), (17408, 1024), (17408, 2048)]
BATCH_GROUPS = [(768, 512, 12), (2048, 512, 12)]   # the 110M model's attention and down_proj layers
PEAK_FP32_TFLOPS = 157.3     # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E


# kernel families of one call: (name, spanqr_profile_kernel id, launches per call)
FAMILIES = [("amax", _lib.K_AMAX, 1), ("gram_pass1", _lib.K_GRAM_PASS1, 1), ("gram", _lib.K_GRAM, 4),
            ("reduce", _lib.K_REDUCE, 5), ("chol", _lib.K_CHOL, 3), ("trsm_pass1", _lib.K_TRSM_PASS1, 1),
            ("trsm", _lib.K_TRSM, 2), ("ns_apply", _lib.K_NS_APPLY, 2)]


def algorithmic(family, K, r):
    """(flops, HBM bytes) of one launch at (K, r): Gram K r (r+1) flops (symmetric half) reading X once; solve
    K r (r+1) flops reading A (and Z on pass 1) and writing Y; NS apply 2 K r^2 flops reading Y and writing Q;
    Cholesky r^3 / 3 flops; amax reads X; the reduce moves only r x r partials (not counted)."""
    kr = 4.0 * K * r
    return {"amax": (0.0, kr), "gram_pass1": (K * r * (r + 1.0), kr), "gram": (K * r * (r + 1.0), kr),
            "reduce": (0.0, 0.0), "chol": (r ** 3 / 3.0, 0.0), "trsm_pass1": (K * r * (r + 1.0), 3 * kr),
            "trsm": (K * r * (r + 1.0), 2 * kr), "ns_apply": (2.0 * K * r * r, 2 * kr)}[family]


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
    copy of the kernel (spanqr_profile_chol): list of (step us, of which tile factor + next-row wait us)"""
    K, r = X.shape
    kcholqr_f(X)
    plan = get_plan(K, r, X.device)
    G, npart = stages.gram(X, kahan=True, use_scale=True)
    nb = r // 32
    stamps = (ctypes.c_ulonglong * (6 * nb))()
    tick = ctypes.c_double()
    _lib.check(_lib.lib().spanqr_profile_chol(plan.handle, G.data_ptr(), npart.data_ptr(), 1e-7, 1e-8, stamps,
                                              ctypes.byref(tick), stream_handle(X.device)))
    us = lambda a, b: (stamps[b] - stamps[a]) * tick.value / 1000.0
    return [(us(1 + 4 * j, 1 + 4 * (j + 1)), us(1 + 4 * j, 2 + 4 * j)) for j in range(nb)]


def traffic_bytes(family):
    """HBM bytes per launch of a kernel family at the workload, from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE runs
    recorded in profiles/traffic.json (None if that kernel has no record)"""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            rec = json.load(f).get(family)
    except (OSError, ValueError):
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


def time_replays(graphs, steps, reps=5):
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


def batched_layers(dev, steps):
    """the batched layer set: per training step, orth of 12 layers at 768x512 and 12 at 2048x512 (independent
    inputs of the cond-1e8 generator, seeds 100 + i), as two batched graphs (one per shape group) and as 24
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
    t_single = time_replays([g for g, _q in single], steps)
    t_batched = time_replays([g for g, _q in batched], steps)
    res = {"layers": sum(n for _k, _r, n in BATCH_GROUPS),
           "groups": [f"{n} x {K}x{r}" for K, r, n in BATCH_GROUPS],
           "us_per_step_batched": t_batched, "us_per_step_sequential": t_single,
           "speedup": t_single / t_batched, "bitwise_equal_to_single_calls": same,
           "orth_max": max(orth_error(q) for q in q_batched),
           "chol_per_launch": {f"{K}x{r}": get_plan(K, r, dev, n).chol_batch for K, r, n in BATCH_GROUPS}}
    del single, batched
    torch.cuda.synchronize()
    return res


def orth_error(Q):
    Qd = Q.detach().double().cpu()
    return float((Qd.T @ Qd - torch.eye(Q.shape[1], dtype=torch.float64)).abs().max())


def time_graph(g, n=20, reps=5):
    """median over `reps` bursts of n back-to-back replays, microseconds per replay"""
    out = []
    for _ in range(reps):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        s.record()
        for _ in range(n):
            g.replay()
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e) * 1000.0 / n)
    return statistics.median(out)


def lat_us(g, n=20):
    """isolated synchronised call: median host wall time of one replay followed by a device synchronisation"""
    out = []
    torch.cuda.synchronize()
    for _ in range(n):
        t0 = time.perf_counter()
        g.replay()
        torch.cuda.synchronize()
        out.append((time.perf_counter() - t0) * 1e6)
    return statistics.median(out)


def kernels_at(X, reps):
    """per kernel family at X's shape: average launch duration and its algorithmic rates"""
    K, r = X.shape
    out = {}
    for fam, which, per_call in FAMILIES:
        us = kernel_avg_us(X, which, reps)
        fl, by = algorithmic(fam, K, r)
        out[fam] = {"us": us, "per_call": per_call, "tflops": fl / us / 1e6, "gbs": by / us / 1e3,
                    "mfma_frac": fl / us / 1e6 / PEAK_FP32_TFLOPS, "hbm_frac": by / us / 1e3 / PEAK_HBM_GBS}
    return out


def cpu_baseline(inputs, seconds):
    """the oracle (C restatement, OpenMP) and CPU torch.linalg.qr on the host, on a bounded sample"""
    import oracle
    threads = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    torch.set_num_threads(threads)
    per_shape, hh = {}, {}
    budget = seconds / max(1, len(inputs))
    for (K, r), X in inputs.items():
        Xn = X.cpu().numpy()
        KS = get_plan(K, r, X.device).split_rows
        oracle.orth(Xn, KS)                                  # warm-up
        times, t_end = [], time.perf_counter() + budget
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            oracle.orth(Xn, KS)
            times.append(time.perf_counter() - t0)
        per_shape[f"{K}x{r}"] = statistics.median(times) * 1e6
        Xc = X.cpu()
        torch.linalg.qr(Xc)
        ht = []
        for _ in range(5):
            t0 = time.perf_counter()
            torch.linalg.qr(Xc)
            ht.append(time.perf_counter() - t0)
        hh[f"{K}x{r}"] = statistics.median(ht) * 1e6
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            model = next((l.split(":", 1)[1].strip() for l in f if l.startswith("model name")), "")
    except OSError:
        pass
    return {
        "value": statistics.mean(per_shape.values()), "unit": "us/call", "cores": threads, "kind": "port",
        "sample": f"oracle/kcholf_oracle.c orth() on seed 0 of each workload shape, >= {budget:.1f} s each, median",
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
    a = p.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py measures one GPU: orth() of one matrix runs on a single MI355X and this build has no "
              f"multi-GPU path, so --gpus {a.gpus} is not supported", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    inputs = {}
    for K, r in WORKLOAD_SHAPES:
        for s in SEEDS:
            inputs[(K, r, s)] = gen.ttf_uu(K, r, N=K, seed=s).to(dev)
    if a.no_graph:
        class _Direct:
            def __init__(self, X):
                self.X = X
                self.Q = kcholqr_f(X)

            def replay(self):
                self.Q = kcholqr_f(self.X)

        graphs = {}
        for key, X in inputs.items():
            d = _Direct(X)
            graphs[key] = (d, d.Q)
    else:
        graphs = {key: capture(X) for key, X in inputs.items()}
    for _ in range(a.warmup):
        for g, _q in graphs.values():
            g.replay()
    torch.cuda.synchronize()
    calls = len(graphs)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(a.steps):
        for g, _q in graphs.values():
            g.replay()
    end.record()
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(end)
    value = total_ms * 1000.0 / (a.steps * calls)
    orth_max = max(orth_error(q) for _g, q in graphs.values())

    per_shape, per_shape_lat = {}, {}
    for (K, r, s), (g, _q) in graphs.items():
        per_shape.setdefault(f"{K}x{r}", []).append(time_graph(g))
        per_shape_lat.setdefault(f"{K}x{r}", []).append(lat_us(g))
    per_shape = {k: statistics.mean(v) for k, v in per_shape.items()}
    per_shape_lat = {k: statistics.mean(v) for k, v in per_shape_lat.items()}
    shapes = {}
    for K, r in OTHER_SHAPES:
        X = gen.bench_input(K, r, seed=0).to(dev)
        g, q = capture(X) if not a.no_graph else (lambda d: (d, d.Q))(_Direct(X))
        ks = kernels_at(X, a.kernel_reps)
        shapes[f"{K}x{r}"] = {"thr_us": time_graph(g), "lat_us": lat_us(g), "orth": orth_error(q),
                              "sum_of_kernels_us": sum(v["us"] * v["per_call"] for v in ks.values()),
                              "kernels": ks}
        del g, q, X
        torch.cuda.synchronize()
    blocked = {}
    for K, r in BLOCKED_SHAPES:
        X = gen.bench_input(K, r, seed=0).to(dev)
        g, q = capture(X, orth)
        blocked[f"{K}x{r}"] = {"thr_us": time_graph(g, n=5), "lat_us": lat_us(g, n=5), "orth": orth_error(q),
                               "blocks": r // 256, "orth_calls_per_call": 2 * (r // 256) - 1}
        del g, q, X
        torch.cuda.synchronize()
    # fp64 clamped Cholesky with fp32 copies (kchol.chol64; not on orth's path): HIP events around back-to-back calls
    chol64 = {}
    for n in (256, 512):
        Xd = torch.randn(n + 64, n, device=dev, dtype=torch.float64, generator=torch.Generator(dev).manual_seed(n))
        G64 = Xd.T @ Xd
        for _ in range(2):
            kchol.chol64(G64, 1e-12)
        s_, e_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s_.record()
        for _ in range(10):
            kchol.chol64(G64, 1e-12)
        e_.record()
        torch.cuda.synchronize()
        chol64[str(n)] = {"us": s_.elapsed_time(e_) * 100.0}
        del Xd, G64
    targets = {k: {"us_per_call": shapes[k]["thr_us"], "lat_us": shapes[k]["lat_us"], "orth": shapes[k]["orth"],
                   "target_us": TARGET_US[k]} for k in TARGET_US}

    batched = batched_layers(dev, max(1, min(a.steps, 20)))

    # per kernel: average launch duration at each workload shape (HIP events around back-to-back launches)
    kernels = {}
    call_us = {}
    for K, r in WORKLOAD_SHAPES:
        ks = kernels_at(inputs[(K, r, 0)], a.kernel_reps)
        for fam, v in ks.items():
            kernels.setdefault(fam, {})[f"{K}x{r}"] = v
        call_us[f"{K}x{r}"] = sum(v["us"] * v["per_call"] for v in ks.values())
    share = {fam: sum(v[s_]["us"] * v[s_]["per_call"] for s_ in v) / sum(call_us.values())
             for fam, v in kernels.items()}
    dom = max(share, key=share.get)
    dk = kernels[dom]
    avg_us = statistics.mean(v["us"] for v in dk.values())
    fl = statistics.mean(algorithmic(dom, K, r)[0] for K, r in WORKLOAD_SHAPES)
    by = statistics.mean(algorithmic(dom, K, r)[1] for K, r in WORKLOAD_SHAPES)
    bound = "mfma" if fl / PEAK_FP32_TFLOPS >= by / PEAK_HBM_GBS * 1e-3 else "hbm"
    achieved = fl / avg_us / 1e6 if bound == "mfma" else by / avg_us / 1e3
    peak = PEAK_FP32_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
    roofline = {"bound": bound, "kernel": dom, "achieved": achieved, "peak": peak,
                "unit": "TFLOP/s" if bound == "mfma" else "GB/s", "frac": achieved / peak,
                "traffic": traffic_bytes(dom), "avg_launch_us": avg_us, "share_of_call": share[dom],
                "note": "algorithmic work per launch / average launch duration (HIP events around back-to-back "
                        "launches on the call's stream); the Cholesky is latency-bound (its critical path is a chain "
                        "of r pivots), so its roofline fraction is small by construction"}
    call_roof = {}
    for K, r in WORKLOAD_SHAPES:
        F, B = call_work(K, r)
        t = per_shape[f"{K}x{r}"] * 1e-6
        call_roof[f"{K}x{r}"] = {"tflops": F / t / 1e12, "mfma_frac": F / t / 1e12 / PEAK_FP32_TFLOPS,
                                 "gbs": B / t / 1e9, "hbm_frac": B / t / 1e9 / PEAK_HBM_GBS}
    steps = chol_steps_us(inputs[(WORKLOAD_SHAPES[0][0], WORKLOAD_SHAPES[0][1], 0)])
    chol_info = {"r": WORKLOAD_SHAPES[0][1], "us_per_32col_step": [round(a, 2) for a, _ in steps],
                 "us_factor_and_wait": [round(b, 2) for _, b in steps],
                 "us_per_32col_diag_step": statistics.mean(a for a, _ in steps),
                 "note": "device wall clock stamped by workgroup 0 of an instrumented copy of the kernel"}

    cpu = None if a.no_cpu else cpu_baseline({(K, r): inputs[(K, r, 0)] for K, r in WORKLOAD_SHAPES}, a.cpu_seconds)
    line = {
        "metric": METRIC, "value": value, "unit": "us/call", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": total_ms / a.steps, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "0.8B TTF layers: orth() at 1024x256, 2048x256, 3584x256, 2 seeds each, one "
                               "hipGraph per input", "shapes": [f"{K}x{r}" for K, r in WORKLOAD_SHAPES],
                   "seeds": list(SEEDS), "calls_per_step": calls, "graphs": not a.no_graph},
        "orth_max": orth_max, "per_shape_us": per_shape, "per_shape_lat_us": per_shape_lat,
        "target_shapes": targets, "shapes": shapes, "blocked_shapes": blocked, "batched_layers": batched,
        "chol64": chol64,
        "roofline": roofline, "call_roofline": call_roof, "kernels": kernels, "kernel_share": share,
        "sum_of_kernels_us": call_us, "cholesky": chol_info,
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
