"""Program for rocprofv3 counter runs (FETCH_SIZE, WRITE_SIZE): a plain elementwise copy of known size, to scale the
counters, then one warm orth() call per 0.8B workload shape (each kernel of the call dispatched once per shape).

    rocprofv3 --pmc FETCH_SIZE -d OUT -o fetch -- python3 -m spanqr_amd.qrbench.traffic
    rocprofv3 --pmc WRITE_SIZE -d OUT -o write -- python3 -m spanqr_amd.qrbench.traffic
    python3 -m spanqr_amd.qrbench.rocprof_summary traffic OUT/fetch_counter_collection.csv \\
        OUT/write_counter_collection.csv
"""
import sys

import torch

COPY_FLOATS = 1 << 27          # 512 MiB read + 512 MiB written: twice the 256 MB last-level cache
SHAPES = [(1024, 256), (2048, 256), (3584, 256)]


def main():
    from spanqr_amd import kcholqr_f
    from spanqr_amd.qrbench import gen
    dev = torch.device("cuda:0")
    a = torch.ones(COPY_FLOATS, device=dev)
    b = torch.empty_like(a)
    torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    del a, b
    for K, r in SHAPES:
        X = gen.ttf_uu(K, r, N=K, seed=0).to(dev)
        kcholqr_f(X)
        torch.cuda.synchronize()
        print(f"traffic: orth {K}x{r}", flush=True)
        kcholqr_f(X)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
