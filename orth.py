"""spanqr entry point (drop-in for the reference's orth.py:1-20).

    from orth import orth
    Q = orth(X)          # X: fp32 GPU [K, r] -> Q: fp32 [K, r], orthonormal columns, span(Q) = span(X)
    Qs = orth_many(Xs)   # the same for a list of layers, batched per shape group (not in the reference)

orth.py:9-10 imports borth and kcholqr_f into the module; they are importable from here too.
"""
from spanqr_amd import borth, kcholqr_f, orth, orth_many  # noqa: F401

__all__ = ["orth", "orth_many", "borth", "kcholqr_f"]
