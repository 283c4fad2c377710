"""kchol.chol32(G, tau) (candidates/kchol.py:35-44) through spanqr_chol32: L and Li bit-identical to the oracle's
clamped factorisation, tau given as a float or as a device tensor (read on the device, no host synchronisation), only
G's lower triangle read, G left intact, zeros above L's diagonal, and a strided G."""
import numpy as np
import pytest
import torch

import oracle
from spanqr_amd import kchol
from spanqr_amd.qrbench import gen

from checks import assert_bits

pytestmark = pytest.mark.gpu


def spd(n, seed, cond_scale=1e-7):
    """a shifted Gram of a benchmark-like X (fp32, symmetric)"""
    X = gen.ttf_uu(max(n, 64), n, seed=seed).double()
    G = X.T @ X
    G = G + cond_scale * torch.linalg.matrix_norm(G) * torch.eye(n, dtype=torch.float64)
    return G.float().numpy()


@pytest.mark.parametrize("n", [32, 128, 256, 512, 544, 1024])
@pytest.mark.parametrize("tau_on_device", [False, True])
def test_chol32_bit_exact(cuda, n, tau_on_device):
    print(f"chol32 n={n} device tau={tau_on_device}", flush=True)
    G = spd(n, seed=n)
    tau = np.float32(1e-4 * np.abs(G).max())
    Gd = torch.from_numpy(G).to(cuda)
    G0 = Gd.clone()
    t = torch.tensor([tau], device=cuda) if tau_on_device else float(tau)
    L, Li = kchol.chol32(Gd, t)
    Lo, Lio = oracle.chol(G, tau)
    assert_bits(L, Lo, "L (zeros above the diagonal included)")
    assert_bits(Li, Lio, "Li")
    assert_bits(Gd, G0, "G left intact")


def test_chol32_clamps_and_reads_lower_triangle(cuda):
    """a rank-deficient G whose clamped pivots take tau from a device tensor, with NaN written above the diagonal:
    only the lower triangle is read (kchol.py:37)"""
    n = 256
    rng = np.random.default_rng(5)
    B = rng.standard_normal((n, n // 2)).astype(np.float64)
    G = (B @ B.T).astype(np.float32)
    # a floor well above the rounding noise of the deficient half keeps the clamped factor's tile inverses finite (a
    # floor near the noise level makes them overflow, on the GPU and in the oracle alike)
    tau = np.float32(1e-2 * np.abs(G).max())
    Gn = G.copy()
    Gn[np.triu_indices(n, 1)] = np.nan
    L, Li = kchol.chol32(torch.from_numpy(Gn).to(cuda), torch.tensor(tau, device=cuda))
    Lo, Lio = oracle.chol(G, tau)
    assert np.isfinite(Lo).all() and np.isfinite(Lio).all()
    d = np.diag(Lo)
    assert (d[n // 2 + 8:] == np.float32(tau) * oracle.rsqrt(np.float32(tau))).all(), "the deficient half is clamped"
    assert_bits(L, Lo, "L")
    assert_bits(Li, Lio, "Li")
    assert np.isfinite(L.cpu().numpy()).all()


def test_chol32_strided_g(cuda):
    n, pad = 512, 36
    G = spd(n, seed=3)
    Gp = torch.full((n, n + pad), float("nan"), device=cuda)
    Gp[:, :n] = torch.from_numpy(G).to(cuda)
    tau = np.float32(1e-5 * np.abs(G).max())
    L, Li = kchol.chol32(Gp[:, :n], float(tau))
    Lo, Lio = oracle.chol(G, tau)
    assert_bits(L, Lo, "L from a strided G")
    assert_bits(Li, Lio, "Li from a strided G")


def test_chol32_rejects_bad_arguments(cuda):
    with pytest.raises(ValueError):
        kchol.chol32(torch.zeros(48, 48, device=cuda), 1e-6)
    with pytest.raises(TypeError):
        kchol.chol32(torch.zeros(64, 64, device=cuda, dtype=torch.float64), 1e-6)
    with pytest.raises(TypeError):
        kchol.chol32(torch.zeros(64, 64), 1e-6)
