"""spanqr_amd: spanqr's orth(X) -- a robust shifted Cholesky-QR for tall fp32 matrices -- on AMD MI355X (gfx950).

    from orth import orth          # drop-in, as in the reference (orth.py)
    Q = orth(X)                    # X: fp32 GPU [K, r] -> Q: fp32 [K, r], Q^T Q = I, span(Q) = span(X)

The hot path is hand-written HIP in csrc/spanqr.hip behind the C ABI of include/spanqr.h, loaded with ctypes.
"""
from .kcholqr import borth, kcholqr_f, kcholqr_f_many, orth, orth_many, set_checked, status  # noqa: F401
from .plan import clear_plans, get_plan  # noqa: F401

__all__ = ["orth", "orth_many", "kcholqr_f", "kcholqr_f_many", "borth", "get_plan", "clear_plans", "set_checked",
           "status"]
