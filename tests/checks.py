"""Shared assertions of the GPU tests: bitwise equality with a readable diff, and the spec's robustness gates."""
import numpy as np
import torch

from spanqr_amd.qrbench import metrics


def assert_bits(a, b, what):
    a = a.detach().cpu().numpy() if isinstance(a, torch.Tensor) else a
    b = b.detach().cpu().numpy() if isinstance(b, torch.Tensor) else b
    same = np.array_equal(np.ascontiguousarray(a).view(np.uint32), np.ascontiguousarray(b).view(np.uint32))
    if not same:
        d = np.abs(a.astype(np.float64) - b.astype(np.float64))
        raise AssertionError(f"{what}: {int((a.view(np.uint32) != b.view(np.uint32)).sum())} elements differ, "
                             f"max abs diff {np.nanmax(d):.3e}")


def gate(X, Q, what, orth_tol=metrics.ORTH_TOL_TARGET):
    """the spec's robustness gates: no collapsed columns, max|Q^T Q - I| <= orth_tol (2e-7 unless given), the
    reference's span rule"""
    ref = metrics.reference(X)
    res = metrics.assess(Q, X.to(Q.device), ref)
    hh = metrics.assess(metrics.householder(X.cpu()), X.cpu(), ref)
    fails = res.failures(span_ref=hh.span_n, orth_tol=orth_tol)
    assert not fails, f"{what}: {fails} (orth {res.orth:.3e}, span_n {res.span_n:.2f})"
