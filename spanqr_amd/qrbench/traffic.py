"""Program for rocprofv3 counter runs at the target shapes: a plain elementwise copy of known size (to scale the byte
counters), then for each shape two orth() calls (the second, warm one is the one summarised), each kernel of a call
dispatched once.

    rocprofv3 --pmc FETCH_SIZE -d OUT -o fetch -- python3 -m spanqr_amd.qrbench.traffic
    rocprofv3 --pmc WRITE_SIZE -d OUT -o write -- python3 -m spanqr_amd.qrbench.traffic
    rocprofv3 --pmc SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES SQ_BUSY_CYCLES -d OUT -o mfma -- python3 -m ...traffic
    python3 -m spanqr_amd.qrbench.rocprof_summary traffic OUT/fetch_counter_collection.csv \\
        OUT/write_counter_collection.csv --json profiles/traffic.json
"""
import sys

import torch

COPY_FLOATS = 1 << 27          # 512 MiB read + 512 MiB written: twice the 256 MB last-level cache
# (name, K, r, N of the generator): the shapes the targets are quoted at
SHAPES = [("768x512", 768, 512, 768), ("17408x256", 17408, 256, 5120)]


def main():
    from spanqr_amd import kcholqr_f
    from spanqr_amd.qrbench import gen
    dev = torch.device("cuda:0")
    a = torch.ones(COPY_FLOATS, device=dev)
    b = torch.empty_like(a)
    torch.mul(a, 1.0, out=b)
    torch.cuda.synchronize()
    del a, b
    for name, K, r, N in SHAPES:
        X = gen.ttf_uu(K, r, N=N, seed=0).to(dev)
        kcholqr_f(X)
        torch.cuda.synchronize()
        print(f"traffic: orth {name}", flush=True)
        kcholqr_f(X)
        torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
