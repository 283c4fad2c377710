"""The fp64 clamped Cholesky (kchol.chol64 -> chol_f64) through the C ABI: L, Li and their fp32 copies bit-identical
to the oracle's fp64 restatement at n = 32..1024 on SPD, rank-deficient, zero and NaN-pivot inputs, tau as a float or
a device tensor, repeat determinism, and no wait that gave up."""
import numpy as np
import pytest
import torch

import oracle
from spanqr_amd import kchol

pytestmark = pytest.mark.gpu


def _bits(a, b, what):
    """bit-identical, except that a NaN matches any NaN: the default NaN differs between the host (sign set) and the
    GPU (canonical positive), and a clamped NaN pivot with a tiny tau overflows into NaNs further down"""
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    u = np.uint64 if a.dtype == np.float64 else np.uint32
    both_nan = np.isnan(a) & np.isnan(b)
    diff = (np.ascontiguousarray(a).view(u) != np.ascontiguousarray(b).view(u)) & ~both_nan
    assert not diff.any(), f"{what}: {int(diff.sum())} elements differ"


def _case(n, kind, rng):
    if kind == "spd":
        X = rng.standard_normal((n + 50, n)) * np.exp(rng.uniform(-4, 4, n))
        return X.T @ X, 1e-14
    if kind == "rank":
        B = rng.standard_normal((n, n // 4))
        return B @ B.T, 1e-9
    if kind == "zero":
        return np.zeros((n, n)), 1e-30
    X = rng.standard_normal((n + 10, n))
    G = X.T @ X
    G[n // 3, n // 3] = np.nan
    return G, 1e-6


@pytest.mark.parametrize("n,kind", [(32, "spd"), (64, "spd"), (128, "rank"), (256, "spd"), (256, "nan"),
                                    (512, "spd"), (512, "zero"), (1024, "spd")])
def test_chol64_bit_exact(cuda, n, kind):
    rng = np.random.default_rng(n + len(kind))
    G, tau = _case(n, kind, rng)
    print(f"chol64 n={n} {kind}", flush=True)
    L, Li, Lf, Lif = kchol.chol64(torch.from_numpy(G).to(cuda), tau)
    kchol.status(n, cuda)
    Lo, Lio, Lfo, Lifo = oracle.chol64(G, tau)
    _bits(L, Lo, "L")
    _bits(Li, Lio, "Li")
    _bits(Lf, Lfo, "Lf")
    _bits(Lif, Lifo, "Lif")


def test_chol64_tau_tensor_and_repeat(cuda):
    rng = np.random.default_rng(3)
    X = rng.standard_normal((300, 256))
    G = torch.from_numpy(X.T @ X).to(cuda)
    t = torch.tensor([1e-12], device=cuda, dtype=torch.float64)
    a = kchol.chol64(G, t)
    b = kchol.chol64(G, 1e-12)
    c = kchol.chol64(G, t)
    torch.cuda.synchronize()
    for x, y, z in zip(a, b, c):
        assert torch.equal(x, y) and torch.equal(x, z)
    L = a[0].cpu().numpy()
    assert np.abs(L @ L.T - X.T @ X).max() <= 1e-12 * np.abs(X.T @ X).max()


def test_chol64_rejects_bad_inputs(cuda):
    with pytest.raises(TypeError):
        kchol.chol64(torch.zeros(64, 64, device=cuda), 1e-9)          # fp32
    with pytest.raises(ValueError):
        kchol.chol64(torch.zeros(48, 48, device=cuda, dtype=torch.float64), 1e-9)
    with pytest.raises(ValueError):
        kchol.chol64(torch.zeros(1056, 1056, device=cuda, dtype=torch.float64), 1e-9)
