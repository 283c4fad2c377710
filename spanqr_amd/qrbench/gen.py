"""Test matrices for orth(X), restated from qrbench/gen.py (reference) plus the MI355X benchmark generators.

Reference cases (qrbench/gen.py:53-164) are built exactly as the reference builds them: fp64 on the CPU from a
seeded torch.Generator, then rounded to fp32. The seed formula is gen.py:179. The `cond` column of the reference's
saved runs (results/synth_kcholf.json) fingerprints these inputs, so a matching cond proves the same X was rebuilt.

Benchmark generator (`ttf_uu`): X = V (U^T U) + u^T U, the TTF update shape. V [K, r] orthonormal (Q of a QR of a
seeded N(0,1) matrix), U = A diag(s) B^T [N, r] with A, B orthonormal and s log-uniform over [1, 10^cu], u [N, K]
N(0,1) scaled to unit RMS (an Adam-normalised gradient). u^T U is accumulated over row chunks of u so the N x K
matrix is never held whole.

All builders return CPU tensors; the caller moves them to the device.
"""
import math
from dataclasses import dataclass, field
from pathlib import Path

import torch

# (K, r) per model (the TTF layers that call orth) -- gen.py:16-22
SHAPES = {
    "110m": [(768, 512), (2048, 512)],
    "0.8b": [(1024, 256), (2048, 256), (3584, 256)],
    "27b": [(5120, 256), (6144, 256), (17408, 256)],
}
BENCH_SHAPES = [(768, 512), (2048, 512), (5120, 256), (17408, 256)]
ALL_SHAPES = sorted({s for v in SHAPES.values() for s in v})


@dataclass
class Case:
    name: str
    X: torch.Tensor                            # fp32 CPU [K, r], contiguous
    ctx: dict = field(default_factory=dict)    # optional structure (V: previous basis)
    hard: bool = True                          # acceptance case (False: extra robustness case)


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _orth64(K, r, g):
    Q, R = torch.linalg.qr(torch.randn(K, r, generator=g, dtype=torch.float64))
    return Q * torch.sign(torch.diagonal(R))


def _mixed(K, r, s, g):
    return _orth64(K, r, g) @ torch.diag(s) @ _orth64(r, r, g).T


def _finish(X64):
    return X64.to(torch.float32).contiguous()


# ---- reference acceptance / robustness builders (gen.py:53-133) ----

def mixed(K, r, g, c):
    return _mixed(K, r, torch.logspace(0, -c, r, dtype=torch.float64), g)


def cluster(K, r, g, c):
    s = torch.ones(r, dtype=torch.float64)
    s[r // 2:] = 10.0 ** -c
    return _mixed(K, r, s[torch.randperm(r, generator=g)], g)


def zero(K, r, g):
    return torch.zeros(K, r, dtype=torch.float64)


def rank(K, r, g, k):
    return torch.randn(K, k, generator=g, dtype=torch.float64) @ torch.randn(k, r, generator=g, dtype=torch.float64)


def dup_cols(K, r, g):
    X = torch.randn(K, r, generator=g, dtype=torch.float64)
    X[:, r // 2: 2 * (r // 2)] = X[:, : r // 2]
    return X


def zero_block(K, r, g):
    X = torch.randn(K, r, generator=g, dtype=torch.float64)
    X[:, r // 4: r // 2] = 0
    return X


def graded(K, r, g, c):
    return torch.randn(K, r, generator=g, dtype=torch.float64) * torch.logspace(0, -c, r, dtype=torch.float64)


def _ttf_parts(K, r, g, cu, tilt, sig_rank=32, noise=0.3):
    su = torch.logspace(0, -cu, r, dtype=torch.float64)
    Qr = _orth64(r, r, g)
    N = max(K, r)
    Qn = _orth64(N, r, g)
    U_rs = torch.diag(su) @ Qr.T
    B = U_rs.T @ U_rs
    V = _orth64(K, r, g)
    Lf = torch.randn(N, sig_rank, generator=g, dtype=torch.float64) / math.sqrt(N)
    R = torch.randn(K, sig_rank, generator=g, dtype=torch.float64)
    P = R @ ((Lf.T @ Qn) @ U_rs) + noise * torch.randn(K, r, generator=g, dtype=torch.float64) @ U_rs
    VB = V @ B
    if tilt > 0:
        P = P * (tilt * VB.norm() / P.norm())
    else:
        P = torch.zeros_like(P)
    return V, B, P, VB


def ttf_dense(K, r, g, cu, tilt):
    V, B, P, VB = _ttf_parts(K, r, g, cu, tilt)
    return VB + P, {"V": V}


def ttf_first(K, r, g, noise):
    N = max(K, r)
    Lf = torch.randn(N, 32, generator=g, dtype=torch.float64) / math.sqrt(N)
    R = torch.randn(K, 32, generator=g, dtype=torch.float64)
    G = torch.randn(N, r, generator=g, dtype=torch.float64)
    X = R @ (Lf.T @ G)
    if noise > 0:
        X = X + noise * math.sqrt(32) * torch.randn(K, r, generator=g, dtype=torch.float64)
    return X


def _cases_for(K, r):
    """(name, builder(g), hard) in the reference's order (gen.py:138-164); the index feeds the seed"""
    out = []
    for c in (2, 4, 6, 8):
        out.append((f"mixed_c{c}", lambda g, c=c: mixed(K, r, g, c), True))
    out += [
        ("zero", lambda g: zero(K, r, g), True),
        ("rank_half", lambda g: rank(K, r, g, r // 2), True),
        ("dup_cols", lambda g: dup_cols(K, r, g), True),
        ("ttf_cu2_t1e-1", lambda g: ttf_dense(K, r, g, 2, 1e-1), True),
        ("ttf_cu4_t1e-2", lambda g: ttf_dense(K, r, g, 4, 1e-2), True),
        ("ttf_cu4_t1", lambda g: ttf_dense(K, r, g, 4, 1.0), True),
        ("ttf_zero_grad_cu4.5", lambda g: ttf_dense(K, r, g, 4.5, 0.0), True),
        ("ttf_first", lambda g: ttf_first(K, r, g, 0.1), True),
        ("ttf_first_rank32", lambda g: ttf_first(K, r, g, 0.0), True),
        ("mixed_c10", lambda g: mixed(K, r, g, 10), False),
        ("mixed_c14", lambda g: mixed(K, r, g, 14), False),
        ("cluster_c5", lambda g: cluster(K, r, g, 5), False),
        ("cluster_c9", lambda g: cluster(K, r, g, 9), False),
        ("zero_block", lambda g: zero_block(K, r, g), False),
        ("rank_1", lambda g: rank(K, r, g, 1), False),
        ("graded_c8", lambda g: graded(K, r, g, 8), False),
        ("tiny_1e-25", lambda g: 1e-25 * mixed(K, r, g, 4), False),
        ("huge_1e25", lambda g: 1e25 * mixed(K, r, g, 4), False),
    ]
    return out


def case_names(K=768, r=512):
    return [n for n, _, _ in _cases_for(K, r)]


def case_seed(K, r, index, s):
    """gen.py:179"""
    return 1_000_003 * s + 7919 * index + K * 31 + r


def make_cases(K, r, names=None, seeds=(0,), include_extra=True):
    """yields Case objects (gen.py:171-182); names: case names or prefixes (None: all)"""
    for i, (name, build, hard) in enumerate(_cases_for(K, r)):
        if names and not any(name == n or name.startswith(n) for n in names):
            continue
        if not hard and not include_extra and not names:
            continue
        for s in seeds:
            out = build(_gen(case_seed(K, r, i, s)))
            X64, ctx = out if isinstance(out, tuple) else (out, {})
            yield Case(f"{name}/s{s}", _finish(X64), {k: _finish(v) for k, v in ctx.items()}, hard)


# ---- benchmark generator: X = V (U^T U) + u^T U ----

def ttf_uu(K, r, N=None, seed=0, cu=4.0, chunk=512):
    """X = V (U^T U) + u^T U (see module docstring). cond(U^T U) reaches 10^(2 cu) (1e8 at cu = 4)."""
    N = K if N is None else N
    g = _gen(seed)
    V = _orth64(K, r, g)
    A = _orth64(N, r, g)
    B = _orth64(r, r, g)
    s = 10.0 ** (cu * torch.rand(r, generator=g, dtype=torch.float64))
    U = (A * s) @ B.T                                        # [N, r]
    uU = torch.zeros(K, r, dtype=torch.float64)
    ss = 0.0
    for n0 in range(0, N, chunk):
        uc = torch.randn(min(chunk, N - n0), K, generator=g, dtype=torch.float64)
        ss += float((uc * uc).sum())
        uU += uc.T @ U[n0:n0 + uc.shape[0]]
    uU /= math.sqrt(ss / (N * K))                           # u scaled to unit RMS
    return _finish(V @ (U.T @ U) + uU)


def bench_input(K, r, seed=0):
    """the benchmark's input at (K, r): ttf_uu with N = K, except N = 5120 for the 27B shapes (K >= 5120)"""
    return ttf_uu(K, r, N=5120 if K >= 5120 else K, seed=seed)


# ---- adversarial set (cond 1e14, rank 1, zeroed half, duplicated columns, zero, 1e+-25 scaling) ----

def adversarial(K, r, seed=0):
    """dict name -> fp32 X"""
    g = _gen(10_007 + seed)
    out = {}
    out["cond1e14"] = _finish(_mixed(K, r, torch.logspace(0, -14, r, dtype=torch.float64), g))
    a = torch.randn(K, 1, generator=g, dtype=torch.float64)
    b = torch.randn(1, r, generator=g, dtype=torch.float64)
    out["rank1"] = _finish(a @ b)
    X = torch.randn(K, r, generator=g, dtype=torch.float64)
    X[:, r // 2:] = 0
    out["right_half_zero"] = _finish(X)
    X = torch.randn(K, r, generator=g, dtype=torch.float64)
    X[:, r - 64:] = X[:, :64]
    out["dup64"] = _finish(X)
    out["zero"] = torch.zeros(K, r, dtype=torch.float32)
    base = ttf_uu(K, r, seed=seed).double()
    out["cond1e8_x1e-25"] = _finish(base * 1e-25)
    out["cond1e8_x1e25"] = _finish(base * 1e25)
    return out


# ---- matrices dumped from a training run (qrbench/gen.py:185-194) ----

def real_cases(dump_dir="dumps", shape=None):
    """Case per *.pt file under dump_dir (recursively, sorted), as written by spanqr_amd.qrbench.dump or the
    reference's qrbench.dump: a dict with 'X' and optionally 'V' (the previous basis, kept in ctx), or a bare tensor.
    shape: only files whose X is [K, r] = shape. Loaded with torch.load(weights_only=True); CPU fp32 tensors."""
    root = Path(dump_dir)
    for p in sorted(root.rglob("*.pt")):
        d = torch.load(p, map_location="cpu", weights_only=True)
        X = d["X"] if isinstance(d, dict) else d
        if shape is not None and tuple(X.shape) != tuple(shape):
            continue
        ctx = {}
        if isinstance(d, dict) and d.get("V") is not None:
            ctx["V"] = d["V"].float().contiguous()
        yield Case(f"real/{p.relative_to(root).with_suffix('')}", X.float().contiguous(), ctx, True)
