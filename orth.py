"""spanqr entry point (drop-in for the reference's orth.py:1-20).

    from orth import orth
    Q = orth(X)          # X: fp32 GPU [K, r] -> Q: fp32 [K, r], orthonormal columns, span(Q) = span(X)
"""
from spanqr_amd import orth  # noqa: F401

__all__ = ["orth"]
