"""Benchmark of orth(X) on one MI355X: microseconds per orth() call, max|Q^T Q - I|, and the roofline of each kernel.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--cpu-seconds S]

Workload (the reference's 0.8B TTF layer shapes): K x r in {1024x256, 2048x256, 3584x256}, two seeds each, X = V (U^T U)
+ u^T U with N = K (U's singular values log-uniform over [1, 1e4], u unit-RMS Gaussian), generated on the CPU and
resident on the GPU before timing. One step = one orth() call on each of the six inputs; every input has its own
captured hipGraph. `value` = timed wall time / (steps x 6) in microseconds (lower is better).

Also reported: per-shape back-to-back time, the 768x512 and 17408x256 shapes (quoted targets), the per-kernel profile
(HIP events recorded after every kernel of one call, on the call's stream) with algorithmic flops and bytes per
kernel, and a CPU baseline (the C restatement of the algorithm in oracle/, OpenMP, on the host; plus CPU
torch.linalg.qr) on a bounded sample.
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

from spanqr_amd import _lib, kcholqr_f  # noqa: E402
from spanqr_amd.plan import get_plan, stream_handle  # noqa: E402
from spanqr_amd.qrbench import gen  # noqa: E402

METRIC = "µs per orth() call at K×r (median); max|QᵀQ−I|; % of HBM/MFMA roofline"
WORKLOAD_SHAPES = [(1024, 256), (2048, 256), (3584, 256)]
SEEDS = (0, 1)
TARGET_SHAPES = [(768, 512), (17408, 256)]
PEAK_FP32_TFLOPS = 157.3     # MI355X dense fp32 matrix
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E
KERNELS = (["amax"] + [f"{k}{p}" for p in range(1, 4) for k in ("gram", "reduce", "chol", "trsm")]
           + [f"ns_{k}{i}" for i in range(1, 3) for k in ("gram", "reduce", "apply")])


def algorithmic(name, K, r):
    """(flops, bytes) per launch of kernel `name` at (K, r): the per-unit figures of one orth() call, split by
    kernel. Gram: K r (r+1) flops (symmetric), reads X once; TRSM: K r (r+1) flops, reads A (and Z on pass 1),
    writes Y; NS apply: 2 K r^2 flops, reads Y, writes Q; Cholesky: r^3/3 flops; amax reads X; reduce: overhead."""
    kr = 4.0 * K * r
    if name == "amax":
        return 0.0, kr
    if name.startswith("gram") or name.startswith("ns_gram"):
        return float(K) * r * (r + 1), kr
    if name.startswith("trsm"):
        return float(K) * r * (r + 1), (3 if name == "trsm1" else 2) * kr
    if name.startswith("ns_apply"):
        return 2.0 * K * r * r, 2 * kr
    if name.startswith("chol"):
        return r ** 3 / 3.0, 0.0
    return 0.0, 0.0


def family(name):
    for f in ("ns_gram", "ns_reduce", "ns_apply", "gram", "reduce", "chol", "trsm", "amax"):
        if name.startswith(f):
            return f
    return name


def profile_call(X):
    """per-kernel milliseconds of one orth() call on the current stream (events after every kernel)"""
    K, r = X.shape
    plan = get_plan(K, r, X.device)
    Q = torch.empty_like(X)
    ms = (ctypes.c_float * 64)()
    n = ctypes.c_int()
    _lib.check(_lib.lib().spanqr_profile_orth(plan.handle, X.data_ptr(), r, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2,
                                              stream_handle(X.device), ms, 64, ctypes.byref(n)))
    return list(ms[:n.value])


def capture(X):
    """(graph, Q): one orth() call on X captured into a hipGraph on a side stream (plan created beforehand)"""
    st = torch.cuda.Stream(X.device)
    st.wait_stream(torch.cuda.current_stream(X.device))
    with torch.cuda.stream(st):
        kcholqr_f(X)               # creates the plan for this stream and warms up
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=st):
        Q = kcholqr_f(X)
    torch.cuda.synchronize()
    return g, Q


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
    a = p.parse_args(argv)
    if a.gpus != 1:
        print(f"bench.py runs on one GPU: orth() on a single MI355X is the benchmark; --gpus {a.gpus} is not "
              "supported (see DESIGN.md for how the work would shard)", file=sys.stderr)
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

    per_shape = {}
    for (K, r, s), (g, _q) in graphs.items():
        per_shape.setdefault(f"{K}x{r}", []).append(time_graph(g))
    per_shape = {k: statistics.mean(v) for k, v in per_shape.items()}
    targets = {}
    for K, r in TARGET_SHAPES:
        X = gen.bench_input(K, r, seed=0).to(dev)
        g, q = capture(X) if not a.no_graph else (lambda d: (d, d.Q))(_Direct(X))
        targets[f"{K}x{r}"] = {"us_per_call": time_graph(g), "orth": orth_error(q)}
        del g

    # per-kernel profile over the workload inputs (events on the call's stream)
    fam_ms, fam_n, fam_flops, fam_bytes, kern = {}, {}, {}, {}, {}
    for (K, r, s), X in inputs.items():
        ms = [statistics.median(v) for v in zip(*[profile_call(X) for _ in range(5)])]
        for name, t in zip(KERNELS, ms):
            f = family(name)
            fl, by = algorithmic(name, K, r)
            fam_ms[f] = fam_ms.get(f, 0.0) + t
            fam_n[f] = fam_n.get(f, 0) + 1
            fam_flops[f] = fam_flops.get(f, 0.0) + fl
            fam_bytes[f] = fam_bytes.get(f, 0.0) + by
            kern.setdefault(name, []).append(t * 1000.0)
    stages = {}
    for f in fam_ms:
        secs = fam_ms[f] / 1000.0
        stages[f] = {"us_per_launch": fam_ms[f] * 1000.0 / fam_n[f], "share": fam_ms[f] / sum(fam_ms.values()),
                     "tflops": fam_flops[f] / secs / 1e12, "gbs": fam_bytes[f] / secs / 1e9,
                     "mfma_frac": fam_flops[f] / secs / 1e12 / PEAK_FP32_TFLOPS,
                     "hbm_frac": fam_bytes[f] / secs / 1e9 / PEAK_HBM_GBS}
    dom = max(fam_ms, key=fam_ms.get)
    ds = stages[dom]
    roofline = {"bound": "mfma", "kernel": dom, "achieved": ds["tflops"], "peak": PEAK_FP32_TFLOPS,
                "unit": "TFLOP/s", "frac": ds["mfma_frac"], "traffic": None,
                "note": "algorithmic flops per launch / average launch time from HIP events on the call's stream"}

    cpu = None if a.no_cpu else cpu_baseline({(K, r): inputs[(K, r, 0)] for K, r in WORKLOAD_SHAPES}, a.cpu_seconds)
    line = {
        "metric": METRIC, "value": value, "unit": "us/call", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": total_ms / a.steps, "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "0.8B TTF layers: orth() at 1024x256, 2048x256, 3584x256, 2 seeds each, one "
                               "hipGraph per input", "shapes": [f"{K}x{r}" for K, r in WORKLOAD_SHAPES],
                   "seeds": list(SEEDS), "calls_per_step": calls, "graphs": not a.no_graph},
        "orth_max": orth_max, "per_shape_us": per_shape, "target_shapes": targets,
        "roofline": roofline, "stages": stages,
        "kernels_us": {k: statistics.mean(v) for k, v in kern.items()},
        "cpu_baseline": cpu,
        "device": torch.cuda.get_device_name(dev),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
