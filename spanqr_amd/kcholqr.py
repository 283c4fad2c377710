"""orth(X) on MI355X: the robust shifted Cholesky-QR of candidates/kcholqr.py:92-112 ("kcholf") through the native
library. The signature and keyword arguments are the reference's; the whole call is enqueued on the current stream
with no host synchronisation.
"""
import ctypes
import os

import torch

from . import _lib
from .plan import get_borth_plan, get_plan, stream_handle

CB = 32          # Cholesky tile (chol.cu:15 TB = 32)
TILE = 32        # the native kernels need r to be a multiple of this (kcholqr.py:98-99, TB = 32)
R_MAX = 512      # orth.py:18: wider X goes through block Gram-Schmidt in the reference
BLOCK = 256      # its block width (orth.py:19, borth(X, 256))
KCHOLF_MAX_R = 1024   # full-width kcholf (orth.py:20 for r > 512 not a multiple of 256; chol.cu:1 takes n <= ~1024)


def _full_width(K, r):
    """kcholf at full width natively: r a multiple of 32 up to 1024, K >= r"""
    return r % TILE == 0 and r <= KCHOLF_MAX_R and K >= r


def _blocked(r):
    """orth.py:18: above 512 columns a multiple of 256 goes through borth over 256-column blocks"""
    return r > R_MAX and r % BLOCK == 0


# Opt-in check of the Cholesky's bounded waits. The reference launches its Cholesky cooperatively (kchol.py:43), so a
# launch that cannot be co-scheduled fails loudly there; here a wait that gives up (another kernel holding the CUs
# for ~1 s) makes that matrix's Q NaN without a host synchronisation. With checking on (set_checked(True), or the
# environment variable SPANQR_CHECK=1 at import), every call synchronises afterwards and raises SpanqrError instead.
_CHECKED = [os.environ.get("SPANQR_CHECK", "") == "1"]


def set_checked(on=True):
    """turn the per-call status check on or off (off by default: it costs a host synchronisation per call); returns
    the previous setting"""
    prev = _CHECKED[0]
    _CHECKED[0] = bool(on)
    return prev


def _after(plan):
    if _CHECKED[0]:
        plan.status()


def status(X):
    """raise SpanqrError if the last native call on X's shape (on X's device and the current stream) had a Cholesky
    wait that gave up; X: the tensor, or a list of same-shape tensors as passed to kcholqr_f_many. Synchronises."""
    Xs = list(X) if isinstance(X, (list, tuple)) else [X]
    K, r = Xs[0].shape
    dev = Xs[0].device
    if _blocked(r) and len(Xs) == 1:
        return get_borth_plan(K, r, BLOCK, True, dev).status()
    return get_plan(K, r, dev, min(len(Xs), _lib.MAX_BATCH)).status()


def _check_input(X):
    if not isinstance(X, torch.Tensor) or X.dim() != 2:
        raise ValueError("orth: X must be a 2-D tensor [K, r]")
    if X.dtype != torch.float32:
        raise TypeError(f"orth: X must be float32, got {X.dtype}")
    if X.device.type != "cuda":
        raise TypeError("orth: X must be on a GPU (ROCm device); the hot path has no CPU implementation")


def _prepare(X):
    """contiguous (kcholqr.py:100) and 16-byte aligned (a view with an odd storage offset is copied)"""
    X = X.contiguous()
    if X.data_ptr() % 16:
        X = X.clone()
    return X


def kcholqr_f(X, eps=5e-7, alpha=1e-7, tau=1e-8, ns=2):
    """Q = orth(X) for fp32 X [K, r] on a ROCm device, r a multiple of 32 in [32, 1024] (at full width, also where
    orth takes borth), K >= r (candidates/kcholqr.py:92-112). eps: dust scale (first solve only); alpha:
    diagonal shift relative to ||G||_F; tau: pivot clamp relative to ||G||_F (plus 1e-30); ns: Newton-Schulz polish
    steps (the last with a Kahan Gram).
    """
    _check_input(X)
    K, r = X.shape
    if not _full_width(K, r):
        raise ValueError(f"kcholqr_f: shape [{K}, {r}] needs r % {TILE} == 0, r <= {KCHOLF_MAX_R} and K >= r")
    X = _prepare(X)
    dev = X.device
    plan = get_plan(K, r, dev)
    Q = torch.empty_like(X)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().spanqr_orth_f32(plan.handle, X.data_ptr(), r, Q.data_ptr(), r, float(eps), float(alpha),
                                               float(tau), int(ns), stream_handle(dev)))
    _after(plan)
    return Q


def kcholqr_f_many(Xs, eps=5e-7, alpha=1e-7, tau=1e-8, ns=2):
    """[kcholqr_f(X) for X in Xs] for same-shape fp32 matrices on one device, in launches that cover up to
    32 matrices each (one kernel per stage for the whole group; the Cholesky in groups that fit the device at once).
    Every Q is bit-identical to kcholqr_f on that X alone. No counterpart in the reference, whose optimizer calls
    orth once per layer (qrbench/methods.py:47-50).
    """
    Xs = list(Xs)
    if not Xs:
        return []
    for X in Xs:
        _check_input(X)
    K, r = Xs[0].shape
    dev = Xs[0].device
    for X in Xs:
        if tuple(X.shape) != (K, r) or X.device != dev:
            raise ValueError("kcholqr_f_many: every X must have the same shape and device")
    if not _full_width(K, r):
        raise ValueError(f"kcholqr_f_many: shape [{K}, {r}] needs r % {TILE} == 0, r <= {KCHOLF_MAX_R} and K >= r")
    Xs = [_prepare(X) for X in Xs]
    Qs = [torch.empty_like(X) for X in Xs]
    n_all = len(Xs)
    plan = get_plan(K, r, dev, min(n_all, _lib.MAX_BATCH))
    with torch.cuda.device(dev):
        for i0 in range(0, n_all, plan.batch):
            xs, qs = Xs[i0:i0 + plan.batch], Qs[i0:i0 + plan.batch]
            n = len(xs)
            xp = (ctypes.c_void_p * n)(*[x.data_ptr() for x in xs])
            qp = (ctypes.c_void_p * n)(*[q.data_ptr() for q in qs])
            _lib.check(_lib.lib().spanqr_orth_batched_f32(plan.handle, n, xp, r, qp, r, float(eps), float(alpha),
                                                          float(tau), int(ns), stream_handle(dev)))
            _after(plan)
    return Qs


def orth_many(Xs):
    """[orth(X) for X in Xs] with the matrices grouped by shape and device: each group of native shapes runs as
    batched launches (kcholqr_f_many), so the latency-bound Cholesky of a group costs about as much as one. Results
    come back in input order and are bit-identical to orth(X) on each X.
    """
    Xs = list(Xs)
    out = [None] * len(Xs)
    groups = {}
    for i, X in enumerate(Xs):
        _check_input(X)
        K, r = X.shape
        if _full_width(K, r) and not _blocked(r):
            groups.setdefault((K, r, X.device), []).append(i)
        else:
            out[i] = orth(X)
    for idx in groups.values():
        for i, Q in zip(idx, kcholqr_f_many([Xs[i] for i in idx])):
            out[i] = Q
    return out


def borth(X, b=512, reorth=True):
    """Q for fp32 X [K, r], K >= r, by block Gram-Schmidt over b-column blocks (candidates/kbig.py:69-95, BCGS2, with
    the reference's signature and defaults): each block, scaled by the power of 2 of the whole X, has the finished
    blocks' span removed twice and goes through the kcholf recipe with its own column slice of a K x r dust; with
    reorth it is projected and orthonormalised once more. One native call for the whole X, no host synchronisation.

    As kbig.py:77-78, r <= b or r not a multiple of b is one kcholf call at full width instead (here for r a multiple
    of 32 up to 1024; other such shapes use torch.linalg.qr). Natively b is a multiple of 32 in
    [32, 1024] (orth passes 256, the reference's default is 512); other b raise ValueError, as does r above 4096.
    """
    _check_input(X)
    K, r = X.shape
    if r <= b or r % b:
        if _full_width(K, r):
            return kcholqr_f(X)
        return torch.linalg.qr(X)[0]
    if b % TILE or not TILE <= b <= KCHOLF_MAX_R:
        raise ValueError(f"borth: b = {b}: the native block width must be a multiple of {TILE} in [{TILE}, "
                         f"{KCHOLF_MAX_R}]")
    if r > _lib.MAX_R or K < r:
        raise ValueError(f"borth: shape [{K}, {r}] needs r <= {_lib.MAX_R} and K >= r")
    X = _prepare(X)
    dev = X.device
    plan = get_borth_plan(K, r, b, reorth, dev)
    Q = torch.empty_like(X)
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().spanqr_orth_f32(plan.handle, X.data_ptr(), r, Q.data_ptr(), r, 5e-7, 1e-7, 1e-8, 2,
                                               stream_handle(dev)))
    _after(plan)
    return Q


def orth(X):
    """Orthonormal basis of the column span of X (fp32 GPU [K, r], K >= r), as orth.py:13-20: Q^T Q = I and
    span(Q) = span(X); rank-deficient or zero X is completed with orthonormal directions (never zero or NaN columns).
    Deterministic and free of host synchronisation.

    Dispatch as orth.py:18-20: r > 512 and a multiple of 256 goes through block Gram-Schmidt over 256-column blocks
    (borth); any other r that is a multiple of 32 through kcholqr_f at full width. Shapes outside the native kernels
    -- r not a multiple of 32 (kcholqr.py:98-99, as the reference) and, here, K < r, r > 4096, or r > 1024 and not a
    multiple of 256 (where the reference's kcholqr_f would run a Cholesky wider than its chol.cu:1 bound) -- go to
    torch.linalg.qr.
    """
    _check_input(X)
    K, r = X.shape
    if _blocked(r):
        if r <= _lib.MAX_R and K >= r:
            return borth(X, BLOCK)
        return torch.linalg.qr(X)[0]
    if not _full_width(K, r):
        return torch.linalg.qr(X)[0]
    return kcholqr_f(X)
